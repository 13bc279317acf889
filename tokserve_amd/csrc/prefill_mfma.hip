// Chunked-prefill paged attention with MFMA for both products, bf16/fp16, block
// sizes that are multiples of 16 (keys move in 16-key pages).
//
// One workgroup (4 waves) per (sequence, KV head, tile of QT query tokens). The
// tile's rows are (token, query head) pairs, row = token * G + head, 128 rows
// per workgroup, RT 16-row tiles per wave. Keys are processed 32 at a time
// (two pages). Per step every wave computes, per 16-row tile,
//
//   S^T (32 keys x 16 rows) = K . Q^T          2 x (Dh/32) v_mfma_f32_16x16x32
//     A = K rows from LDS, B = Q^T held in registers for the whole kernel;
//     lane (g, r) receives keys g*4 + i (+16 for the second page) of row r,
//   online softmax per row (running max / sum kept per lane for its row),
//   O^T (Dh x 16 rows) += V^T . P^T            (Dh/16) v_mfma_f32_16x16x32
//     B = P^T straight from the S^T accumulators, A = V^T.
//
// K and V pages move HBM -> LDS with global_load_lds_dwordx4 (16 bytes per lane
// written straight into LDS, no registers) into a three-stage ring, two steps
// ahead of the compute. Rows keep their natural [key][dim] layout with the 16-byte
// chunks of each row XOR-swizzled (Swizzle below), so that neither operand read
// has LDS bank conflicts. V^T operands come from the same
// layout through ds_read_b64_tr_b16: within each 16-lane group, result element e
// of lane j is element j % 4 of the 8 bytes that lane 4e + j / 4 addressed, so a
// lane addressing dims 4c .. 4c+3 of key m hands dim j of keys 0..3 to lane j.
//
// All LDS reads of a step are issued in one inline-asm block that ends with its
// own wait (compiled for the device only; the host pass sees no body): the
// compiler, which cannot tell the LDS ring stages apart, would
// otherwise wait for every outstanding HBM -> LDS load before each LDS read.
// The step barrier is likewise explicit and waits only for the loads of the
// step about to be read.
//
// The causal mask is key <= query position, query i of sequence b sitting at
// seq_lens[b] - q_len_b + i (tokserve/kernels/_triton_paged_attention.py:118-123).
#include "attention_common.hpp"

namespace tks {
namespace {

constexpr int kPWaves = 4;
constexpr int kXcds = 8;  // MI355X: 8 accelerator dies, workgroups dealt round-robin
constexpr int kKeysPerStep = 32;
// LDS ring stages. Dh 128 runs its steps in pairs over 4 stages: the wait for
// the next pair's loads and the workgroup barrier come once per pair, and the
// second step's K tile is read right behind the first step's PV MFMAs; the
// next pair loads meanwhile. Dh 64 keeps 3 stages (steps s+1 and s+2 load while
// step s computes, one barrier per step) so that 4 workgroups fit a CU's LDS.
template <int DH>
constexpr bool kPairSteps = DH == 128;
template <int DH>
constexpr int kStagesOf = kPairSteps<DH> ? 4 : 3;

// Makes a wave-uniform value an SGPR that is ready here: every scalar load
// behind it completes before this point, so no wait for such a load can land
// inside the main loop (a scalar-load wait also waits for all pending LDS
// reads, which would serialise the loop's LDS pipeline).
template <typename V>
__device__ __forceinline__ void settle_sgpr(V &v) {
#if __HIP_DEVICE_COMPILE__
  asm volatile("" : "+s"(v));
#endif
}

// Orders the computation of v before the asm statements that follow (a
// volatile asm that takes v as an operand; it emits nothing).
template <typename V>
__device__ __forceinline__ void pin_vgpr(V &v) {
#if __HIP_DEVICE_COMPILE__
  asm volatile("" : "+v"(v));
#endif
}

// Waits until at most N of this wave's vector-memory operations are
// outstanding, then joins the workgroup barrier.
template <int N>
__device__ __forceinline__ void wait_loads_and_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

#define TKS_S(x) #x
#define TKS_RD128(o, a, off) "ds_read_b128 %" TKS_S(o) ", %" TKS_S(a) " offset:%" TKS_S(off) "\n\t"
#define TKS_RDTR(o, a, off) "ds_read_b64_tr_b16 %" TKS_S(o) ", %" TKS_S(a) " offset:%" TKS_S(off) "\n\t"
#define TKS_RD32(o, a, off) "ds_read_b32 %" TKS_S(o) ", %" TKS_S(a) " offset:" TKS_S(off) "\n\t"

// LDS reads of one step, issued without waiting: K operands k[kt * NC + c]
// (rows kt*16 + r) of a stage, and V^T halves v[d * 2 + page] plus the block
// ids of a later step. O0 is the byte offset of the ring stage, O1 = O0 + 16
// rows (the second page). The results are valid only after lds_wait(...) on
// them: the wait is a separate asm statement that names the same registers,
// so nothing reads them before it.
template <int DH>
struct StepReads;

template <>
struct StepReads<128> {
  static constexpr int kRows16 = 16 * 128 * 2;  // bytes of 16 rows
  template <int O0, int O1>
  static __device__ __forceinline__ void keys(const uint32_t (&ka)[4], u32x4 (&k)[8]) {
    static_assert(O1 == O0 + kRows16 && O1 < 65536, "offsets");
#if __HIP_DEVICE_COMPILE__
    asm volatile(
        TKS_RD128(0, 8, 12) TKS_RD128(1, 9, 12) TKS_RD128(2, 10, 12) TKS_RD128(3, 11, 12)
        TKS_RD128(4, 8, 13) TKS_RD128(5, 9, 13) TKS_RD128(6, 10, 13) TKS_RD128(7, 11, 13)
        : "=&v"(k[0]), "=&v"(k[1]), "=&v"(k[2]), "=&v"(k[3]), "=&v"(k[4]), "=&v"(k[5]),
          "=&v"(k[6]), "=&v"(k[7])
        : "v"(ka[0]), "v"(ka[1]), "v"(ka[2]), "v"(ka[3]), "i"(O0), "i"(O1)
        : "memory");
#endif
  }
  template <int O0, int O1>
  static __device__ __forceinline__ void values(const uint32_t (&va)[8], uint32_t ba, u32x2 (&v)[16],
                                                uint32_t (&bid)[2]) {
    static_assert(O1 == O0 + kRows16 && O1 < 65536, "offsets");
#if __HIP_DEVICE_COMPILE__
    asm volatile(
        TKS_RDTR(0, 18, 27) TKS_RDTR(1, 18, 28) TKS_RDTR(2, 19, 27) TKS_RDTR(3, 19, 28)
        TKS_RDTR(4, 20, 27) TKS_RDTR(5, 20, 28) TKS_RDTR(6, 21, 27) TKS_RDTR(7, 21, 28)
        TKS_RDTR(8, 22, 27) TKS_RDTR(9, 22, 28) TKS_RDTR(10, 23, 27) TKS_RDTR(11, 23, 28)
        TKS_RDTR(12, 24, 27) TKS_RDTR(13, 24, 28) TKS_RDTR(14, 25, 27) TKS_RDTR(15, 25, 28)
        TKS_RD32(16, 26, 0) TKS_RD32(17, 26, 4)
        : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
          "=&v"(v[6]), "=&v"(v[7]), "=&v"(v[8]), "=&v"(v[9]), "=&v"(v[10]), "=&v"(v[11]),
          "=&v"(v[12]), "=&v"(v[13]), "=&v"(v[14]), "=&v"(v[15]), "=&v"(bid[0]), "=&v"(bid[1])
        : "v"(va[0]), "v"(va[1]), "v"(va[2]), "v"(va[3]), "v"(va[4]), "v"(va[5]), "v"(va[6]),
          "v"(va[7]), "v"(ba), "i"(O0), "i"(O1)
        : "memory");
#endif
  }
  static __device__ __forceinline__ void wait_keys(u32x4 (&k)[8]) {
#if __HIP_DEVICE_COMPILE__
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(k[0]), "+v"(k[1]), "+v"(k[2]), "+v"(k[3]), "+v"(k[4]), "+v"(k[5]),
                   "+v"(k[6]), "+v"(k[7])::"memory");
#endif
  }
  static __device__ __forceinline__ void wait_values(u32x2 (&v)[16], uint32_t (&bid)[2]) {
#if __HIP_DEVICE_COMPILE__
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]),
                   "+v"(v[6]), "+v"(v[7]), "+v"(v[8]), "+v"(v[9]), "+v"(v[10]), "+v"(v[11]),
                   "+v"(v[12]), "+v"(v[13]), "+v"(v[14]), "+v"(v[15]), "+v"(bid[0]),
                   "+v"(bid[1])::"memory");
#endif
  }
};

template <>
struct StepReads<64> {
  static constexpr int kRows16 = 16 * 64 * 2;
  template <int O0, int O1>
  static __device__ __forceinline__ void keys(const uint32_t (&ka)[2], u32x4 (&k)[4]) {
    static_assert(O1 == O0 + kRows16 && O1 < 65536, "offsets");
#if __HIP_DEVICE_COMPILE__
    asm volatile(TKS_RD128(0, 4, 6) TKS_RD128(1, 5, 6) TKS_RD128(2, 4, 7) TKS_RD128(3, 5, 7)
                 : "=&v"(k[0]), "=&v"(k[1]), "=&v"(k[2]), "=&v"(k[3])
                 : "v"(ka[0]), "v"(ka[1]), "i"(O0), "i"(O1)
                 : "memory");
#endif
  }
  template <int O0, int O1>
  static __device__ __forceinline__ void values(const uint32_t (&va)[4], uint32_t ba, u32x2 (&v)[8],
                                                uint32_t (&bid)[1]) {
    static_assert(O1 == O0 + kRows16 && O1 < 65536, "offsets");
#if __HIP_DEVICE_COMPILE__
    asm volatile(
        TKS_RDTR(0, 9, 14) TKS_RDTR(1, 9, 15) TKS_RDTR(2, 10, 14) TKS_RDTR(3, 10, 15)
        TKS_RDTR(4, 11, 14) TKS_RDTR(5, 11, 15) TKS_RDTR(6, 12, 14) TKS_RDTR(7, 12, 15)
        TKS_RD32(8, 13, 0)
        : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
          "=&v"(v[6]), "=&v"(v[7]), "=&v"(bid[0])
        : "v"(va[0]), "v"(va[1]), "v"(va[2]), "v"(va[3]), "v"(ba), "i"(O0), "i"(O1)
        : "memory");
#endif
  }
  static __device__ __forceinline__ void wait_keys(u32x4 (&k)[4]) {
#if __HIP_DEVICE_COMPILE__
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(k[0]), "+v"(k[1]), "+v"(k[2]), "+v"(k[3])::"memory");
#endif
  }
  static __device__ __forceinline__ void wait_values(u32x2 (&v)[8], uint32_t (&bid)[1]) {
#if __HIP_DEVICE_COMPILE__
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]),
                   "+v"(v[6]), "+v"(v[7]), "+v"(bid[0])::"memory");
#endif
  }
};

#undef TKS_RD128
#undef TKS_RDTR
#undef TKS_RD32
#undef TKS_S

template <int N>
struct Const {
  static constexpr int value = N;
};

// XOR swizzles of the 16-byte chunks of a K or V row in LDS, a function of the
// row within its 16-row page (so the second page of a step, read at an
// immediate offset, has the same pattern). Chosen so that neither operand read
// has bank conflicts (64 banks of 4 bytes):
//   K (ds_read_b128, 16 lanes = rows 0..15 at one logical chunk): Dh 128 rows
//     are 256 bytes, so row r takes chunk c ^ r; Dh 64 rows are 128 bytes and
//     rows r, r + 8 share banks, so the chunk index mixes r >> 1 instead.
//   V^T (ds_read_b64_tr_b16, 16 lanes = rows 4g .. 4g+3 x chunks 2d, 2d+1 x
//     two 8-byte halves): Dh 128 takes c ^ 2 (row & 7), which sends the eight
//     (row, chunk) pairs to eight different chunks; Dh 64 takes c ^ row.
template <int DH>
struct Swizzle {
  static __device__ __forceinline__ int k(int row) {
    return DH == 128 ? (row & 15) : ((row >> 1) & 7);
  }
  static __device__ __forceinline__ int v(int row) {
    return DH == 128 ? 2 * (row & 7) : (row & 7);
  }
};

// Waves per SIMD the register budget is cut for: Dh 128 (80 KB of LDS per
// workgroup) runs 2 workgroups per CU, Dh 64 (40 KB) fits 4 in LDS and, at 128
// registers, 4 waves per SIMD (measured 448 -> 372 us on a 63k-token Dh 64 prefill).
template <int DH>
constexpr int kPrefillOccupancy = DH == 64 ? 4 : 2;

template <typename T, int DH, int G, int RT>
__global__ __launch_bounds__(64 * kPWaves) __attribute__((amdgpu_waves_per_eu(
    kPrefillOccupancy<DH>, kPrefillOccupancy<DH>))) void prefill_mfma_kernel(PrefillArgs a) {
  constexpr int ROWS = kPWaves * RT * 16;
  constexpr int QT = ROWS / G;           // query tokens per workgroup
  constexpr int NC = DH / 32;            // QK k-chunks
  constexpr int DT = DH / 16;            // PV output dim tiles
  constexpr int KS = kKeysPerStep;
  constexpr bool kPairs = kPairSteps<DH>;
  constexpr int kStages = kStagesOf<DH>;
  constexpr int CPR = DH / 8;            // 16-byte chunks per key row
  constexpr int TILE = KS * DH;          // elements of one K (or V) step tile
  constexpr int STAGE = 2 * TILE;        // K tile then V tile
  constexpr int LOADS = TILE / 8 / (64 * kPWaves);  // 16-byte loads per thread per tile
  static_assert(LOADS >= 1 && (TILE / 8) % (64 * kPWaves) == 0, "tile");
  static_assert(StepReads<DH>::kRows16 == 16 * DH * (int)sizeof(T), "row offsets");
  static_assert(16 % G == 0 || G % 16 == 0, "rows of a tile must be whole tokens");
  // A load's 64 lanes cover 64 / CPR rows from a multiple of that: one page.
  static_assert(16 % (64 / CPR) == 0, "load rows within a page");
  using M = Mfma<T>;
  typedef typename M::f4 f4;
  typedef typename M::v8 v8;

  __shared__ __attribute__((aligned(16))) T ring[kStages * STAGE];
  __shared__ int32_t bt_s[kPrefillBtWindow];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int r = lane & 15;
  const int g = lane >> 4;

  // XCD-aware work mapping. Workgroup i runs on XCD i % 8, and each XCD has its
  // own L2. All query tiles of one (sequence, KV head) read the same K/V pages
  // in the same order, so they are placed on one XCD and dispatched together
  // (the pages come from HBM once per pair, then from that XCD's L2); pairs are
  // dealt round-robin over the XCDs. Within a pair the later tiles (more keys)
  // start first.
  const int xcd = blockIdx.x % kXcds;
  const int slot = blockIdx.x / kXcds;
  const int pair = (slot / a.tiles) * kXcds + xcd;
  if (pair >= a.num_pairs) return;
  const int tile = a.tiles - 1 - slot % a.tiles;
  const int kvh = pair % a.num_kv_heads;
  const int rank = pair / a.num_kv_heads;
  const int b = a.seq_order ? min(max(a.seq_order[rank], 0), a.num_seqs - 1) : rank;
  const int q0 = a.cu_q[b];
  const int q_len = a.cu_q[b + 1] - q0;
  const int t0 = tile * QT;
  if (t0 >= q_len) return;
  const int kv_len = min(a.seq_lens[b], a.key_cap);
  const int base_pos = kv_len - q_len;  // absolute position of query token 0
  const int t_end = min(q_len, t0 + QT);
  // Keys needed by the last token of the tile (causal); the host keeps key_cap
  // within the LDS block-id window.
  const int n_keys = max(0, min(min(kv_len, base_pos + t_end), kPrefillBtWindow * 16));
  const int n_steps = (n_keys + KS - 1) / KS;
  const int n_pages = (n_keys + 15) / 16;

  const T *q = static_cast<const T *>(a.q);
  T *out = static_cast<T *>(a.out);
  const char *kc = reinterpret_cast<const char *>(static_cast<const T *>(a.kc) + a.pool.layer_base +
                                                  (int64_t)kvh * a.pool.head_stride);
  const char *vc = reinterpret_cast<const char *>(static_cast<const T *>(a.vc) + a.pool.layer_base +
                                                  (int64_t)kvh * a.pool.head_stride);
  // K/V move in pages of 16 keys; a pool block of BS = 16 * ppb keys holds ppb
  // of them per KV head. Page i of the sequence starts at page unit
  // block * (Hkv * ppb) + i % ppb of the layer (unit = 16 rows of one head).
  const int ppb = a.pool.block_size / 16;
  const int units_per_block = (int)(a.pool.block_stride / (16 * DH));
  constexpr int64_t kPageBytes = 16 * DH * (int64_t)sizeof(T);
  const int32_t *bt_row = a.bt + (int64_t)b * a.bt_stride;

  // Page units of the sequence (pages of the last step past the keys map to
  // unit 0: loaded, never used).
  for (int i = tid; i < n_steps * (KS / 16); i += 64 * kPWaves)
    bt_s[i] = i < n_pages ? (int32_t)clamp_block(bt_row[i / ppb], a.pool.num_blocks) * units_per_block + i % ppb
                          : 0;

  // Q^T operands: row tile j of this wave covers rows (wave*RT + j)*16 .. +16.
  v8 qb[RT][NC];
  int qpos[RT];  // absolute position of this lane's row (r) in tile j; -1 = padding
#pragma unroll
  for (int j = 0; j < RT; ++j) {
    const int row = (wave * RT + j) * 16 + r;
    const int t = t0 + row / G;
    const int h = row % G;
    qpos[j] = t < t_end ? base_pos + t : -1;
    const T *qp = q + (int64_t)(q0 + min(t, q_len - 1)) * a.q_ts + (int64_t)(kvh * G + h) * a.q_hs + g * 8;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      uint4 v = t < t_end ? ld16(qp + c * 32) : make_uint4(0, 0, 0, 0);
      qb[j][c] = as_v8<T>(v);
    }
  }
  // Smallest query position among this wave's rows: key steps entirely at or
  // below it (and inside n_keys) need no mask.
  // Padding rows (qpos -1) are left out: their Q^T operands are zero and their
  // results are never stored, so they need no mask.
  int min_pos = 0x7fffffff;
#pragma unroll
  for (int j = 0; j < RT; ++j) min_pos = qpos[j] < 0 ? min_pos : min(min_pos, qpos[j]);
  min_pos = __reduce_min_sync(~0ull, min_pos);
  __syncthreads();  // bt_s ready

  // Load k of wave w fills 16-byte slots (k*kPWaves + w)*64 + lane of a tile;
  // slot = row * CPR + physical chunk. All rows of one load lie in one page.
  auto page_of_load = [&](int step, int k) {
    return step * (KS / 16) + ((k * kPWaves + wave) * 64 / CPR) / 16;
  };
  using Swz = Swizzle<DH>;
  // Byte offsets of this lane's K and V chunks inside their page: LDS slot
  // (row, physical chunk) receives logical chunk physical ^ swizzle(row).
  uint32_t src_off_k[LOADS], src_off_v[LOADS];
#pragma unroll
  for (int k = 0; k < LOADS; ++k) {
    const int slot = (k * kPWaves + wave) * 64 + lane;
    const int row = slot / CPR;
    src_off_k[k] = ((row % 16) * DH + ((slot % CPR) ^ Swz::k(row)) * 8) * (int)sizeof(T);
    src_off_v[k] = ((row % 16) * DH + ((slot % CPR) ^ Swz::v(row)) * 8) * (int)sizeof(T);
  }
  // Issues the loads of one step into ring stage STG; blk[k] is wave-uniform.
  auto issue = [&](auto stage_c, const int32_t (&blk)[LOADS]) {
    constexpr int STG = decltype(stage_c)::value;
#pragma unroll
    for (int k = 0; k < LOADS; ++k) {
      const int slot0 = (k * kPWaves + wave) * 64;
      const int64_t base = (int64_t)__builtin_amdgcn_readfirstlane(blk[k]) * kPageBytes;
      load_lds16(kc + base + src_off_k[k], &ring[STG * STAGE + slot0 * 8]);
      load_lds16(vc + base + src_off_v[k], &ring[STG * STAGE + TILE + slot0 * 8]);
    }
  };

  // Per-lane LDS byte addresses inside stage 0 (stages are immediate offsets).
  const uint32_t ring_base = lds_address(&ring[0]);
  uint32_t ka_addr[NC], va_addr[DT];
#pragma unroll
  for (int c = 0; c < NC; ++c) ka_addr[c] = ring_base + (r * CPR + ((c * 4 + g) ^ Swz::k(r))) * 16;
#pragma unroll
  for (int d = 0; d < DT; ++d) {
    const int row = g * 4 + r / 4;  // + 16 for the second page (immediate offset)
    const int lc = d * 2 + (r % 4) / 2;
    va_addr[d] = ring_base + TILE * (int)sizeof(T) + (row * CPR + (lc ^ Swz::v(row))) * 16 + (r & 1) * 8;
  }
  const uint32_t bt_base = lds_address(&bt_s[0]);

  f4 o[RT][DT];
#pragma unroll
  for (int j = 0; j < RT; ++j)
#pragma unroll
    for (int d = 0; d < DT; ++d) o[j][d] = f4{0.f, 0.f, 0.f, 0.f};
  // Online softmax state of row tile j (row r of the tile in lanes r, r+16,
  // r+32, r+48), with m the reference max in log2 units (-inf before the first
  // finite score): negref = -m (0 while m is -inf, so fully masked rows give
  // p = 0), thr = the raw score above which m must move ((m + 8) / c, -inf
  // exactly while m is), l = this lane's share of the row sum. The reference
  // only moves when a score exceeds it by more than 8 (probabilities stay
  // <= 2^8 meanwhile); until then a step needs no cross-lane max, only each
  // lane's check of its own 8 scores.
  float negref[RT], thr[RT], l[RT];
#pragma unroll
  for (int j = 0; j < RT; ++j) {
    negref[j] = 0.f;
    thr[j] = -INFINITY;
    l[j] = 0.f;
  }

  // Q is in registers before the first HBM -> LDS load, so no wait inside the
  // loop has to count it; likewise the scalars the loop reads.
  float scale_log2 = a.scale_log2;  // > 0 (the host routes other scales elsewhere)
  settle_sgpr(scale_log2);
  settle_sgpr(kc);
  settle_sgpr(vc);
  __builtin_amdgcn_s_waitcnt(0);
  {
    int32_t blk[kStages][LOADS];
#pragma unroll
    for (int i = 0; i < kStages; ++i)
#pragma unroll
      for (int k = 0; k < LOADS; ++k) blk[i][k] = bt_s[min(page_of_load(i, k), kPrefillBtWindow - 1)];
    if (n_steps > 0) issue(Const<0>{}, blk[0]);
    if (n_steps > 1) issue(Const<1>{}, blk[1]);
    if (n_steps > 2) issue(Const<2>{}, blk[2]);
    if constexpr (kStages > 3) {
      if (n_steps > 3) issue(Const<3>{}, blk[3]);
    }
  }
  using Reads = StepReads<DH>;
  constexpr int kStageBytes = STAGE * (int)sizeof(T);
  constexpr int kRowsBytes = 16 * DH * (int)sizeof(T);
  u32x4 kraw[2 * NC];  // K operands of the step about to run
  if (n_steps > 0) {
    // Loads complete in issue order: wait for step 0's (with pairs, steps 0
    // and 1), so that only the later steps' may remain.
    constexpr int kFirst = kPairs ? 2 : 1;
    if (n_steps > kFirst + 1)
      wait_loads_and_barrier<4 * LOADS>();
    else if (n_steps > kFirst)
      wait_loads_and_barrier<2 * LOADS>();
    else
      wait_loads_and_barrier<0>();
    Reads::template keys<0, kRowsBytes>(ka_addr, kraw);
    Reads::wait_keys(kraw);
  }
  // K(s) as MFMA A operands: ka[kt][c] = keys kt*16 + (0..15), dims c*32 + ...
  auto k_operands = [&](v8 (&ka)[2][NC]) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        uint4 u = make_uint4(kraw[kt * NC + c][0], kraw[kt * NC + c][1], kraw[kt * NC + c][2],
                             kraw[kt * NC + c][3]);
        ka[kt][c] = as_v8<T>(u);
      }
  };
  // S^T of row tile j against the keys in ka.
  auto scores = [&](const v8 (&ka)[2][NC], int j, f4 (&t)[2]) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      t[kt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c) t[kt] = M::run(ka[kt][c], qb[j][c], t[kt]);
    }
  };

  // Largest of a lane's 8 scores of one tile (NaN-propagating; a NaN score
  // never moves the reference and yields NaN probabilities, as in softmax).
  auto lane_max = [](const f4 (&t)[2]) {
    const float a0 = nan_max(nan_max(t[0][0], t[0][1]), t[0][2]);
    const float a1 = nan_max(nan_max(t[0][3], t[1][0]), t[1][1]);
    const float a2 = nan_max(nan_max(t[1][2], t[1][3]), a0);
    return nan_max(a1, a2);
  };
  // Probabilities of one tile against its reference: bf16/fp16 MFMA operand,
  // returns the lane's sum of them (fp32, before rounding).
  auto probs = [&](const f4 (&t)[2], float nr, v8 &pb) {
    float p[8];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) p[kt * 4 + i] = fast_exp2(__builtin_fmaf(t[kt][i], scale_log2, nr));
#pragma unroll
    for (int i = 0; i < 8; ++i) pb[i] = static_cast<typename M::elem>(p[i]);
    return ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
  };
  // Moves tile j's reference to the row max when that exceeds it by more than
  // 8 (rare after a row's first keys), rescaling O and l to the new reference.
  auto rebase = [&](int j, float lm) {
    const float mx = xgroup_max(lm) * scale_log2;
    const float m_old = thr[j] == -INFINITY ? -INFINITY : -negref[j];
    const bool bump = mx > m_old + 8.f;
    const float m_new = bump ? mx : m_old;
    const float alpha = bump ? fast_exp2(m_old - m_new) : 1.f;
    negref[j] = m_new == -INFINITY ? 0.f : -m_new;
    thr[j] = (m_new + 8.f) / scale_log2;
    l[j] *= alpha;
#pragma unroll
    for (int d = 0; d < DT; ++d) o[j][d] *= alpha;
  };

  // One step: keys s*KS .. s*KS + KS - 1 from ring stage STG, whose K operands
  // are already in kraw. Pipeline: V(s) LDS reads overlap QK(s) and the
  // softmax; tile 1's QK MFMAs run under tile 0's softmax and tile 0's PV MFMAs
  // under tile 1's probabilities; then K(s+1) is read. With one barrier per
  // step (3 stages), the barrier before that read also frees stage s, which
  // takes the loads of step s+3; with step pairs (4 stages) only the pair's
  // second step waits and joins the barrier, and its stages take the loads of
  // steps s+3 and s+4. Steps whose keys
  // reach past the wave's first query position (or past the last key) apply
  // the causal mask; uniform branches around it keep the unmasked steps free of
  // mask work.
  int32_t blk_pair[LOADS];  // block ids of step s+3, read in the pair's first step s-1
  auto step = [&](auto stage_c, int s) {
    static_assert(RT == 2, "the step interleaves two row tiles");
    constexpr int STG = decltype(stage_c)::value;
    constexpr int O0 = STG * kStageBytes;
    constexpr int N0 = ((STG + 1) % kStages) * kStageBytes;
    // Block ids of the step whose loads this step hands to issue().
    const int ahead = min(s + (kPairs ? 4 : 3), n_steps - 1);
    const uint32_t ba = bt_base + page_of_load(ahead, 0) * 4;
    const bool tail = s * KS + KS > n_keys;
    const bool need_mask = s * KS + KS - 1 > min_pos || tail;
    u32x2 vraw[2 * DT];
    uint32_t bid[LOADS];
    Reads::template values<O0, O0 + kRowsBytes>(va_addr, ba, vraw, bid);

    v8 ka[2][NC];
    k_operands(ka);
    f4 st[RT][2];
    scores(ka, 0, st[0]);
    // Key kp = s*KS + kt*16 + g*4 + i is visible to a row iff kp <= qpos
    // (which also keeps it below n_keys).
    auto mask = [&](int j) {
      const int rel = qpos[j] - (s * KS + g * 4);
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (kt * 16 + i > rel) st[j][kt][i] = -INFINITY;
    };
    v8 pb[RT];
    float ps[RT];
    if (need_mask) mask(0);
    scores(ka, 1, st[1]);
    const float lm0 = lane_max(st[0]);
    bool over = lm0 > thr[0];
    ps[0] = probs(st[0], negref[0], pb[0]);
    // Tile 0's probabilities issue between tile 1's QK MFMAs (one MFMA, then
    // three VALU instructions), and stay here rather than sinking past the
    // rebase branch below.
#pragma unroll
    for (int i = 0; i < 2 * NC; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
    }
    pin_vgpr(pb[0]);
    pin_vgpr(ps[0]);
    if (need_mask) mask(1);
    const float lm1 = lane_max(st[1]);
    over = over || lm1 > thr[1];
    if (__builtin_amdgcn_ballot_w64(over)) {
      rebase(0, lm0);
      rebase(1, lm1);
      ps[0] = probs(st[0], negref[0], pb[0]);
    }

    Reads::wait_values(vraw, bid);
    v8 va[DT];
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      uint4 u = make_uint4(vraw[2 * d][0], vraw[2 * d][1], vraw[2 * d + 1][0], vraw[2 * d + 1][1]);
      va[d] = as_v8<T>(u);
    }
    if (tail) {
      // V rows past the last key hold whatever the pool has there; their
      // probabilities are 0, and 0 * NaN would not be.
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int key = s * KS + (e / 4) * 16 + g * 4 + (e % 4);
        if (key >= n_keys) {
#pragma unroll
          for (int d = 0; d < DT; ++d) va[d][e] = static_cast<typename M::elem>(0.f);
        }
      }
    }
    ps[1] = probs(st[1], negref[1], pb[1]);
#pragma unroll
    for (int j = 0; j < RT; ++j)
#pragma unroll
      for (int d = 0; d < DT; ++d) o[j][d] = M::run(va[d], pb[j], o[j][d]);
    // Tile 1's probabilities issue between tile 0's PV MFMAs.
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
    }

    if (s + 1 < n_steps) {
      if constexpr (kPairs && STG % 2 == 0) {
        // First step of a pair: stage s+1 arrived before the pair's barrier.
        Reads::template keys<N0, N0 + kRowsBytes>(ka_addr, kraw);
#pragma unroll
        for (int k = 0; k < LOADS; ++k) blk_pair[k] = (int32_t)bid[k];
        Reads::wait_keys(kraw);
      } else if constexpr (kPairs) {
        // Second step: the next pair's loads are done and every wave is past
        // its reads of this pair's stages, which take steps s+3 and s+4.
        wait_loads_and_barrier<0>();
        Reads::template keys<N0, N0 + kRowsBytes>(ka_addr, kraw);
        if (s + 3 < n_steps) issue(Const<(STG + 3) % kStages>{}, blk_pair);
        if (s + 4 < n_steps) {
          int32_t blk[LOADS];
#pragma unroll
          for (int k = 0; k < LOADS; ++k) blk[k] = (int32_t)bid[k];
          issue(Const<STG>{}, blk);
        }
        Reads::wait_keys(kraw);
      } else {
        // Step s+1's loads done (only step s+2's may remain), and every wave
        // is past its reads of stage s: K(s+1) can be read and stage s refilled.
        if (s + 2 < n_steps)
          wait_loads_and_barrier<2 * LOADS>();
        else
          wait_loads_and_barrier<0>();
        Reads::template keys<N0, N0 + kRowsBytes>(ka_addr, kraw);
        if (s + 3 < n_steps) {
          int32_t blk[LOADS];
#pragma unroll
          for (int k = 0; k < LOADS; ++k) blk[k] = (int32_t)bid[k];
          issue(Const<STG>{}, blk);
        }
        Reads::wait_keys(kraw);
      }
    }
#pragma unroll
    for (int j = 0; j < RT; ++j) l[j] += ps[j];
  };

  for (int s = 0; s < n_steps; s += kStages) {
    step(Const<0>{}, s);
    if (s + 1 < n_steps) step(Const<1>{}, s + 1);
    if (s + 2 < n_steps) step(Const<2>{}, s + 2);
    if constexpr (kStages > 3) {
      if (s + 3 < n_steps) step(Const<3>{}, s + 3);
    }
  }

  // Row sums over the four lane groups, then O = O^T / l for the valid rows.
#pragma unroll
  for (int j = 0; j < RT; ++j) {
    const float lj = xgroup_sum(l[j]);
    const int row = (wave * RT + j) * 16 + r;
    const int t = t0 + row / G;
    const int h = row % G;
    if (t >= t_end) continue;
    const float inv = (lj > 0.f ? 1.f / lj : 0.f) * a.v_scale;  // v_scale 1: exact no-op
    T *op = out + (int64_t)(q0 + t) * a.o_ts + (int64_t)(kvh * G + h) * a.o_hs + g * 4;
#pragma unroll
    for (int d = 0; d < DT; ++d) {
#pragma unroll
      for (int i = 0; i < 4; ++i) op[d * 16 + i] = from_float<T>(o[j][d][i] * inv);
    }
  }
}

template <typename T>
int32_t launch_typed(const PrefillArgs &a, int32_t num_seqs, int32_t num_kv_heads, int32_t G,
                     int32_t head_dim, int32_t max_query_len, hipStream_t s) {
  constexpr int RT = 2;
  constexpr int ROWS = kPWaves * RT * 16;
#define TKS_PREFILL(DH, GG)                                                                  \
  if (head_dim == DH && G == GG) {                                                           \
    PrefillArgs args = a;                                                                    \
    args.num_kv_heads = num_kv_heads;                                                        \
    args.num_pairs = num_seqs * num_kv_heads;                                                \
    args.tiles = static_cast<int32_t>(ceil_div(max_query_len, ROWS / GG));                   \
    if (args.tiles == 0 || args.num_pairs == 0) return TKS_OK;                               \
    const int64_t groups = ceil_div(args.num_pairs, kXcds);                                  \
    const dim3 grid(static_cast<unsigned>(groups * kXcds * args.tiles), 1, 1);               \
    prefill_mfma_kernel<T, DH, GG, RT><<<grid, 64 * kPWaves, 0, s>>>(args);                  \
    return check_launch();                                                                   \
  }
  TKS_PREFILL(128, 4)
  TKS_PREFILL(128, 8)
  TKS_PREFILL(128, 1)
  TKS_PREFILL(128, 2)
  TKS_PREFILL(128, 16)
  TKS_PREFILL(64, 8)
  TKS_PREFILL(64, 4)
  TKS_PREFILL(64, 2)
  TKS_PREFILL(64, 16)
  TKS_PREFILL(64, 1)
#undef TKS_PREFILL
  return TKS_ERR_VALUE;
}

}  // namespace

bool prefill_mfma_supported(int32_t dtype, int32_t head_dim, int32_t group, int32_t key_cap,
                            int32_t block_size, int64_t num_blocks, int32_t num_kv_heads) {
  if (dtype != TKS_BFLOAT16 && dtype != TKS_FLOAT16) return false;
  if (key_cap > kPrefillBtWindow * 16 || block_size % 16 != 0) return false;
  // Page units (16 rows of one head) of the layer are addressed with 32 bits.
  if (num_blocks * num_kv_heads * (block_size / 16) >= (int64_t{1} << 31)) return false;
  if (head_dim != 64 && head_dim != 128) return false;
  return group == 1 || group == 2 || group == 4 || group == 8 || group == 16;
}

int32_t launch_prefill_mfma(const PrefillArgs &a, int32_t dtype, int32_t num_seqs,
                            int32_t num_kv_heads, int32_t group, int32_t head_dim,
                            int32_t max_query_len, hipStream_t stream) {
  return dtype == TKS_BFLOAT16
             ? launch_typed<bf16_t>(a, num_seqs, num_kv_heads, group, head_dim, max_query_len, stream)
             : launch_typed<_Float16>(a, num_seqs, num_kv_heads, group, head_dim, max_query_len,
                                      stream);
}

}  // namespace tks
