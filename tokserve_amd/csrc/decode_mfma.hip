// Paged decode with MFMA scores, bf16/fp16, block size 16.
//
// One workgroup of NW waves per (sequence, KV head[, split]). The pages of the
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
// Softmax is online per page (running max m, sum l, rescale alpha); the page's
// probabilities (G x 16) go through a per-wave LDS slice. P.V runs on the VALU:
// lane (hg, tg, dc) owns dims dc*8 .. +8 of heads hg*HPL .. +HPL and tokens
// tg*4 .. +3 of every page, so V also arrives as 16-byte loads; the four token
// groups are summed once per wave. Every K/V byte is read from HBM exactly once
// for all G query heads. Pages are double-buffered in registers and a wave's
// block ids sit in one VGPR (broadcast with readlane), so nothing in the page
// loop waits on a dependent memory access.
#include "attention_common.hpp"

namespace tks {
namespace {

constexpr int kWaves = 4;

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

// K/V rows as stored: T itself, or fp8 e4m3 decoded to T (K, exactly: every
// e4m3 value is a bf16 and an f16) or to f32 (V) right after the load. A lane's
// 8 elements are one 16-byte load of T or one 8-byte load of fp8.
template <typename T, typename KV>
struct PageIO {
  typedef uint4 raw;
  static __device__ __forceinline__ raw load(const KV *p) { return ld16_stream(p); }
  static __device__ __forceinline__ typename Mfma<T>::v8 k_operand(raw r) { return as_v8<T>(r); }
  static __device__ __forceinline__ void v_floats(raw r, float *f) { unpack<T>(r, f); }
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
  static __device__ __forceinline__ void v_floats(raw r, float *f) {
    fp8x4_to_float(r.x, f);
    fp8x4_to_float(r.y, f + 4);
  }
};

template <typename T, typename KV, int DH, int G>
__global__ __launch_bounds__(64 * kWaves) void decode_mfma_kernel(DecodeArgs a) {
  using S = DecodeShape<DH, G>;
  constexpr int BS = S::BS, NC = S::NC, LPR = S::LPR, TG = S::TG, HPL = S::HPL;
  using M = Mfma<T>;
  using IO = PageIO<T, KV>;
  using raw = typename IO::raw;
  __shared__ __attribute__((aligned(16))) float p_s[kWaves][G][BS];
  __shared__ __attribute__((aligned(16))) float alpha_s[kWaves][G];
  __shared__ __attribute__((aligned(16))) float m_s[kWaves][G];
  __shared__ __attribute__((aligned(16))) float l_s[kWaves][G];
  __shared__ __attribute__((aligned(16))) float acc_s[kWaves][G][DH];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;   // QK: token of the page
  const int grp = lane >> 4; // QK: k-group / output row block
  const int dc = lane % LPR;          // P.V: 8-dim chunk
  const int tg = (lane / LPR) % TG;   // P.V: token group
  const int hg = lane / (LPR * TG);   // P.V: head group

  const int split = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = a.seq_order ? min(max(a.seq_order[blockIdx.z], 0), (int)gridDim.z - 1)
                            : (int)blockIdx.z;
  // A length above the host bound is clamped so no access can leave its buffer.
  const int len = min(a.seq_lens[b], a.key_cap);
  const int n_pages = (len + BS - 1) / BS;
  const int p_begin = split * a.pages_per_split;
  T *out = static_cast<T *>(a.out);
  if (p_begin >= n_pages) {
    if (split == 0)  // empty sequence: defined all-zero output
      for (int i = threadIdx.x; i < G * DH; i += 64 * kWaves)
        out[b * a.o_ss + (int64_t)(kvh * G + i / DH) * a.o_hs + i % DH] = from_float<T>(0.f);
    return;
  }
  const int p_end = min(n_pages, p_begin + a.pages_per_split);
  const int per_wave = (p_end - p_begin + kWaves - 1) / kWaves;
  const int w_begin = p_begin + wave * per_wave;
  const int w_end = min(p_end, w_begin + per_wave);

  typename M::v8 qa[NC];
  {
    const T *qp = static_cast<const T *>(a.q) + b * a.q_ss + (int64_t)(kvh * G + r % G) * a.q_hs +
                  grp * 8;
#pragma unroll
    for (int c = 0; c < NC; ++c) qa[c] = as_v8<T>(ld16(qp + c * 32));
  }

  const KV *kc = static_cast<const KV *>(a.kc) + a.pool.layer_base + (int64_t)kvh * a.pool.head_stride;
  const KV *vc = static_cast<const KV *>(a.vc) + a.pool.layer_base + (int64_t)kvh * a.pool.head_stride;
  const int k_off = r * DH + grp * 8;
  const int v_off = tg * 4 * DH + dc * 8;
  const int32_t *bt_row = a.bt + (int64_t)b * a.bt_stride;

  float acc[HPL][8];
#pragma unroll
  for (int j = 0; j < HPL; ++j)
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[j][d] = 0.f;
  float m[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.f;
  }

  // Every page is read once: non-temporal loads.
  auto load_page = [&](int blk_reg, int idx, raw (&kr)[NC], raw (&vr)[4]) {
    const int64_t blk = clamp_block(__builtin_amdgcn_readlane(blk_reg, idx), a.pool.num_blocks);
    const KV *kp = kc + blk * a.pool.block_stride + k_off;
    const KV *vp = vc + blk * a.pool.block_stride + v_off;
#pragma unroll
    for (int c = 0; c < NC; ++c) kr[c] = IO::load(kp + c * 32);
#pragma unroll
    for (int j = 0; j < 4; ++j) vr[j] = IO::load(vp + j * DH);
  };

  auto consume = [&](const raw (&kr)[NC], const raw (&vr)[4], int p) {
    typename M::f4 s4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c) s4 = M::run(qa[c], IO::k_operand(kr[c]), s4);
    const bool valid = p * BS + r < len;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float sv = valid ? s4[i] * a.scale_log2 : -INFINITY;
      const float mn = fmaxf(m[i], row16_max(sv));
      const float alpha = fast_exp2(m[i] - mn);
      const float pv = fast_exp2(sv - mn);
      m[i] = mn;
      l[i] = l[i] * alpha + pv;
      const int h = grp * 4 + i;
      if (h < G) {
        p_s[wave][h][r] = pv;
        if (r == 0) alpha_s[wave][h] = alpha;
      }
    }
    wave_lds_sync();
    float vf[4][8];
#pragma unroll
    for (int j = 0; j < 4; ++j) IO::v_floats(vr[j], vf[j]);
    if ((p + 1) * BS > len) {
      // The sequence's last page: rows past the last key hold whatever the pool
      // has there. Their probabilities are 0, and 0 * NaN would not be.
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (p * BS + tg * 4 + j >= len)
#pragma unroll
          for (int d = 0; d < 8; ++d) vf[j][d] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < HPL; ++j) {
      const int h = hg * HPL + j;
      const float al = alpha_s[wave][h];
      const float4 pv = *reinterpret_cast<const float4 *>(&p_s[wave][h][tg * 4]);
#pragma unroll
      for (int d = 0; d < 8; ++d)
        acc[j][d] = acc[j][d] * al + pv.x * vf[0][d] + pv.y * vf[1][d] + pv.z * vf[2][d] +
                    pv.w * vf[3][d];
    }
    wave_lds_sync();
  };

  // Two register pages in flight: the steady-state loop always has the next
  // page's loads issued behind the page being consumed (straight-line, so the
  // wait before each consume covers only its own page); the last one or two
  // pages of a 64-page chunk drain in the epilogue.
  for (int c0 = w_begin; c0 < w_end; c0 += 64) {
    const int n = min(w_end, c0 + 64) - c0;
    const int blk_reg = lane < n ? bt_row[c0 + lane] : 0;
    raw kA[NC], vA[4], kB[NC], vB[4];
    load_page(blk_reg, 0, kA, vA);
    int i = 0;
    for (; i + 2 < n; i += 2) {
      load_page(blk_reg, i + 1, kB, vB);
      consume(kA, vA, c0 + i);
      load_page(blk_reg, i + 2, kA, vA);
      consume(kB, vB, c0 + i + 1);
    }
    if (i + 1 < n) {
      load_page(blk_reg, i + 1, kB, vB);
      consume(kA, vA, c0 + i);
      consume(kB, vB, c0 + i + 1);
    } else {
      consume(kA, vA, c0 + i);
    }
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

template <typename T, typename KV>
int32_t launch_typed(const DecodeArgs &a, int32_t num_seqs, int32_t num_kv_heads, int32_t G,
                     int32_t head_dim, hipStream_t s) {
  const dim3 grid(a.max_splits, num_kv_heads, num_seqs);
#define TKS_DECODE(DH, GG)                                              \
  if (head_dim == DH && G == GG) {                                      \
    decode_mfma_kernel<T, KV, DH, GG><<<grid, 64 * kWaves, 0, s>>>(a);  \
    return check_launch();                                              \
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
