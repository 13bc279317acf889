/*
 * tokserve_hip.h -- C ABI of libtokserve_hip.so, the MI355X (gfx950) kernels of
 * tokserve's continuous-batching hot path: KV append into paged blocks, block
 * table gathers, paged attention (decode and chunked prefill), RMSNorm, RoPE
 * greedy token selection and the elementwise vector_add.
 *
 * Conventions shared by every entry point
 *   - All pointers are device pointers (HBM), except where a comment says host.
 *     The caller owns every buffer; the library never allocates device memory.
 *     Scratch memory (split-K partials) comes in as a caller-owned workspace.
 *   - Sizes and strides are in ELEMENTS, not bytes. The innermost (head_dim or
 *     hidden) dimension must be contiguous.
 *   - `stream` is a hipStream_t (NULL = the default stream). Kernels are only
 *     enqueued; nothing synchronises.
 *   - Return value: TKS_OK (0) or a negative tks_status. The library never
 *     throws across this boundary. A host-side binding maps the codes to the
 *     reference's exception types (ValueError / TypeError / IndexError).
 *   - Paged KV pools use the reference layout [L, NB, Hkv, BS, Dh]
 *     (tokserve/engine/paged/storage.py:40-56), one pool for K and one for V.
 *     A "slot" is block_id * BS + offset (tokserve/engine/paged/block_table.py:53-67).
 *
 * The reference has no compiled code: its kernels are Triton JIT functions in
 * tokserve/kernels/_triton_<op>.py behind the Python wrappers in tokserve/kernels/<op>.py.
 * Each entry point below names the reference interface it replaces.
 */
#ifndef TOKSERVE_HIP_H
#define TOKSERVE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *tks_stream_t; /* hipStream_t */

/* Element types. Values are part of the ABI. */
enum tks_dtype {
  TKS_FLOAT32 = 0,
  TKS_FLOAT16 = 1,
  TKS_BFLOAT16 = 2,
  TKS_FLOAT8_E4M3 = 3, /* OCP e4m3fn (torch.float8_e4m3fn); K/V pools of the *_fp8 entries only */
};

/* Status codes. Values are part of the ABI. */
enum tks_status {
  TKS_OK = 0,
  TKS_ERR_VALUE = -1,     /* shape, size or range error       -> ValueError */
  TKS_ERR_TYPE = -2,      /* unsupported dtype combination    -> TypeError  */
  TKS_ERR_INDEX = -3,     /* layer index out of range         -> IndexError */
  TKS_ERR_WORKSPACE = -4, /* workspace missing or too small   -> ValueError */
  TKS_ERR_LAUNCH = -5,    /* HIP reported a launch error      -> RuntimeError */
};

/* ABI version of this header; bumped on any signature change. */
int32_t tks_abi_version(void);

/* Static description of a status code (never NULL). */
const char *tks_status_string(int32_t status);

/* Message of the last HIP error seen by this thread's last failing call. */
const char *tks_last_hip_error(void);

/* ------------------------------------------------------------------------
 * KV append: scatter new K/V rows into the paged pools.
 * Replaces SequencePagedKVCache.write_layer (tokserve/engine/paged/sequence_cache.py:86-131)
 * and its per-token PagedKVStorage.write_token copies (tokserve/engine/paged/storage.py:64-89).
 *
 * For token t in [0, num_tokens), head h, dim d:
 *   key_cache[layer, slot/BS, h, slot%BS, d] = key[t*key_token_stride + h*key_head_stride + d]
 * (and the same for value), with slot = slot_mapping[t] (int64, device).
 * A negative slot skips the token (padding). Slots >= num_blocks*block_size are
 * never written (callers validate them; the kernel only guards memory).
 * Bit-exact copy.
 */
int32_t tks_kv_append(const void *key, int64_t key_token_stride, int64_t key_head_stride,
                      const void *value, int64_t value_token_stride, int64_t value_head_stride,
                      int64_t num_tokens, void *key_cache, void *value_cache, int32_t num_layers,
                      int64_t num_blocks, int32_t num_kv_heads, int32_t block_size,
                      int32_t head_dim, int32_t layer_index, const int64_t *slot_mapping,
                      int32_t dtype, tks_stream_t stream);

/* ------------------------------------------------------------------------
 * Block-table gather: rebuild logical-order K/V of a ragged batch.
 * Replaces SequencePagedKVCache.read_layer (tokserve/engine/paged/sequence_cache.py:133-193)
 * and PagedKVStorage.read_token (tokserve/engine/paged/storage.py:103-116).
 *
 * For sequence b, position p < seq_lens[b], head h:
 *   key_out[(cu_seqlens[b] + p)*out_token_stride + h*out_head_stride + d]
 *     = key_cache[layer, block_tables[b*block_table_stride + p/BS], h, p%BS, d]
 * block_tables, seq_lens, cu_seqlens are int32 device arrays. Bit-exact copy.
 * max_seq_len (host) must be >= every seq_lens[b].
 */
int32_t tks_paged_gather(const void *key_cache, const void *value_cache, int32_t num_layers,
                         int64_t num_blocks, int32_t num_kv_heads, int32_t block_size,
                         int32_t head_dim, int32_t layer_index, const int32_t *block_tables,
                         int32_t block_table_stride, const int32_t *seq_lens,
                         const int32_t *cu_seqlens, int32_t num_seqs, int32_t max_seq_len,
                         void *key_out, void *value_out, int64_t out_token_stride,
                         int64_t out_head_stride, int32_t dtype, tks_stream_t stream);

/* ------------------------------------------------------------------------
 * Paged attention, decode (one query token per sequence), split-K.
 * Replaces triton_paged_attention for Tq == 1 (tokserve/kernels/paged_attention.py:11-88,
 * kernel tokserve/kernels/_triton_paged_attention.py:12-149), batched over sequences.
 *
 * Query row of sequence b, head hq: query[b*q_seq_stride + hq*q_head_stride + d].
 * It attends to keys 0..seq_lens[b]-1 of KV head hq / (num_q_heads/num_kv_heads)
 * through block_tables[b*block_table_stride + p/BS]:
 *   out = softmax(scale * q.K^T) V, accumulated in fp32, stored in `dtype`.
 * max_seq_len (host) bounds every seq_lens[b] and sizes the grid.
 * pages_per_split: KV blocks per workgroup along the keys (0 = library
 * heuristic: a whole sequence per workgroup when the batch has at least 256
 * (sequence, KV head) pairs, otherwise split so the GPU fills). When some
 * sequence spans more than one split, the partials go to the workspace and a
 * second kernel merges them; the workspace size comes from
 * tks_paged_attention_decode_workspace_bytes with the same arguments (0 when
 * no split is needed; workspace may then be NULL). No initial contents are
 * required. Launches sharing a workspace must be stream-ordered.
 * seq_order (device int32 [num_seqs], may be NULL): the order in which
 * sequences are handed to workgroups, a permutation of 0..num_seqs-1. Passing
 * the sequences longest-first (a host-side plan built from the lengths the
 * scheduler already knows) removes the tail of long sequences started last;
 * results do not depend on it.
 * A sequence with seq_lens[b] == 0 gets an all-zero output row.
 */
int64_t tks_paged_attention_decode_workspace_bytes(int32_t num_seqs, int32_t num_q_heads,
                                                   int32_t num_kv_heads, int32_t head_dim,
                                                   int32_t block_size, int32_t max_seq_len,
                                                   int32_t pages_per_split);

int32_t tks_paged_attention_decode(const void *query, int64_t q_seq_stride, int64_t q_head_stride,
                                   const void *key_cache, const void *value_cache,
                                   int32_t num_layers, int64_t num_blocks, int32_t num_kv_heads,
                                   int32_t block_size, int32_t head_dim, int32_t layer_index,
                                   const int32_t *block_tables, int32_t block_table_stride,
                                   const int32_t *seq_lens, const int32_t *seq_order,
                                   int32_t num_seqs, int32_t num_q_heads,
                                   int32_t max_seq_len, float scale, int32_t pages_per_split,
                                   void *out, int64_t out_seq_stride, int64_t out_head_stride,
                                   void *workspace, int64_t workspace_bytes, int32_t dtype,
                                   tks_stream_t stream);

/* ------------------------------------------------------------------------
 * RoPE, the KV append and decode attention of a decode step in one call.
 * Replaces, for one new token per sequence, the reference's apply_rope
 * (tokserve/engine/rope.py:106-153) of the query and key, write_layer
 * (tokserve/engine/paged/sequence_cache.py:86-131) and triton_paged_attention
 * (tokserve/kernels/paged_attention.py:11-88), which its decode step runs in turn
 * per request (tokserve/engine/attention.py:247-335); in this library, the same as
 * tks_rope_kv_append then tks_paged_attention_decode:
 *   - sequence b's query row (read only; strides q_seq_stride, q_head_stride) is
 *     rotated at positions[b] with the cos/sin tables of tks_rope;
 *   - its new key row (rotated) and value row (strides k_*, v_*, [num_seqs,
 *     num_kv_heads, head_dim]) are written to pool slot slot_mapping[b] of
 *     layer_index, which must address position seq_lens[b] - 1 of sequence b
 *     (a negative slot appends nothing);
 *   - out receives the attention of the rotated query over keys 0..seq_lens[b]-1,
 *     as tks_paged_attention_decode computes it (same workspace rule).
 * Results are bit-identical to the two calls. On the MFMA decode kernel (bf16/fp16
 * rows in 16-byte chunks) this is one launch (plus the split merge): each
 * workgroup rotates its query rows as it loads them, and the wave that reads the
 * sequence's last page uses the new rows in place of what it loads of their slot,
 * then writes them to the pool. Other shapes run the two calls, with the rotated
 * queries staged in `out`.
 */
int32_t tks_rope_append_paged_decode(
    const void *query, int64_t q_seq_stride, int64_t q_head_stride, const void *key,
    int64_t k_seq_stride, int64_t k_head_stride, const void *value, int64_t v_seq_stride,
    int64_t v_head_stride, const int64_t *positions, const void *cos_cache,
    const void *sin_cache, int64_t cache_len, const int64_t *slot_mapping, void *key_cache,
    void *value_cache, int32_t num_layers, int64_t num_blocks, int32_t num_kv_heads,
    int32_t block_size, int32_t head_dim, int32_t layer_index, const int32_t *block_tables,
    int32_t block_table_stride, const int32_t *seq_lens, const int32_t *seq_order,
    int32_t num_seqs, int32_t num_q_heads, int32_t max_seq_len, float scale,
    int32_t pages_per_split, void *out, int64_t out_seq_stride, int64_t out_head_stride,
    void *workspace, int64_t workspace_bytes, int32_t dtype, tks_stream_t stream);

/* ------------------------------------------------------------------------
 * Decode attention that allocates nothing: tks_paged_attention_decode with the
 * split-K partials in a static device buffer the library owns instead of a
 * caller workspace. No counterpart in the reference (whose kernels allocate
 * through torch); it is for callers that cannot allocate device memory: code
 * under HIP graph capture, serving loops and harnesses that forbid hipMalloc.
 *   - Same arguments and results as tks_paged_attention_decode, minus the
 *     workspace. The call makes no hipMalloc / hipFree or allocating library
 *     call.
 *   - The buffer holds at most
 *     tks_paged_attention_decode_noalloc_max_workspace_bytes() bytes (32 MiB);
 *     a batch whose tks_paged_attention_decode_workspace_bytes exceeds it gets
 *     TKS_ERR_WORKSPACE and launches nothing.
 *   - Each GPU holds one copy of the buffer for the life of the process; its
 *     device address is looked up on the first call on each device, with the
 *     calling thread's current device, which must be the device of the stream
 *     and buffers. Every call on a GPU shares that GPU's copy: calls that can
 *     overlap on one GPU (different streams, or threads without ordering) race
 *     and must be serialised by the caller. No initial contents are needed.
 */
int64_t tks_paged_attention_decode_noalloc_max_workspace_bytes(void);

int32_t tks_paged_attention_decode_noalloc(
    const void *query, int64_t q_seq_stride, int64_t q_head_stride, const void *key_cache,
    const void *value_cache, int32_t num_layers, int64_t num_blocks, int32_t num_kv_heads,
    int32_t block_size, int32_t head_dim, int32_t layer_index, const int32_t *block_tables,
    int32_t block_table_stride, const int32_t *seq_lens, const int32_t *seq_order,
    int32_t num_seqs, int32_t num_q_heads, int32_t max_seq_len, float scale,
    int32_t pages_per_split, void *out, int64_t out_seq_stride, int64_t out_head_stride,
    int32_t dtype, tks_stream_t stream);

/* ------------------------------------------------------------------------
 * Paged attention over a ragged batch of query chunks (chunked prefill).
 * Replaces triton_paged_attention for Tq >= 1 with query_position_offset
 * (tokserve/kernels/paged_attention.py:11-88) and the contiguous
 * triton_tiled_attention (tokserve/kernels/tiled_attention.py:9-73).
 *
 * Sequence b owns query tokens cu_seqlens_q[b] .. cu_seqlens_q[b+1]-1 (int32 device
 * array, length num_seqs+1) and seq_lens[b] keys (its KV already appended).
 * Query token i of sequence b sits at absolute position
 *   seq_lens[b] - (cu_seqlens_q[b+1] - cu_seqlens_q[b]) + i
 * and attends causally to keys 0..that position (mask k <= position,
 * tokserve/kernels/_triton_paged_attention.py:118-123).
 * Token n, head hq: query[n*q_token_stride + hq*q_head_stride + d], same for out.
 * num_tokens (host) == cu_seqlens_q[num_seqs]; max_query_len and max_seq_len
 * (host) bound the per-sequence query and key lengths.
 * seq_order (device int32 [num_seqs], may be NULL): the order in which
 * sequences (with all their query tiles) are handed to workgroups, a
 * permutation of 0..num_seqs-1, as for decode. Passing the sequences with the
 * most keys first shortens the tail of long chunks started last; results do
 * not depend on it.
 */
int32_t tks_paged_attention_prefill(const void *query, int64_t q_token_stride,
                                    int64_t q_head_stride, const void *key_cache,
                                    const void *value_cache, int32_t num_layers,
                                    int64_t num_blocks, int32_t num_kv_heads, int32_t block_size,
                                    int32_t head_dim, int32_t layer_index,
                                    const int32_t *block_tables, int32_t block_table_stride,
                                    const int32_t *seq_lens, const int32_t *cu_seqlens_q,
                                    const int32_t *seq_order, int32_t num_seqs, int64_t num_tokens, int32_t num_q_heads,
                                    int32_t max_query_len,
                                    int32_t max_seq_len, float scale, void *out,
                                    int64_t out_token_stride, int64_t out_head_stride,
                                    int32_t dtype, tks_stream_t stream);

/* ------------------------------------------------------------------------
 * fp8 K/V pools (a pool-layout variant behind PagedKVStorage,
 * tokserve/engine/paged/storage.py:40-56, where the reference has only pools in
 * the model dtype). Same layout [L, NB, Hkv, BS, Dh], elements OCP e4m3fn with
 * one fp32 scale per pool (k_scale, v_scale > 0):
 *   stored  = e4m3(clamp(x / scale, -448, 448))   round to nearest even, NaN kept
 *   decoded = float(stored) * scale
 * Each entry takes the arguments of its counterpart above plus the two scales;
 * `dtype` is the type of the non-pool tensors (the new K/V rows, the gathered
 * rows, the query and the output). Attention computes exactly the function of
 * its counterpart on the decoded pools, in fp32, with the scales applied as
 * factors on the scores and on the output.
 */
/* KV append with quantization (tks_kv_append on fp8 pools). */
int32_t tks_kv_append_fp8(const void *key, int64_t key_token_stride, int64_t key_head_stride,
                          const void *value, int64_t value_token_stride,
                          int64_t value_head_stride, int64_t num_tokens, void *key_cache,
                          void *value_cache, int32_t num_layers, int64_t num_blocks,
                          int32_t num_kv_heads, int32_t block_size, int32_t head_dim,
                          int32_t layer_index, const int64_t *slot_mapping, float k_scale,
                          float v_scale, int32_t dtype, tks_stream_t stream);

/* Block-table gather with decoding into `dtype` (tks_paged_gather on fp8 pools). */
int32_t tks_paged_gather_fp8(const void *key_cache, const void *value_cache, int32_t num_layers,
                             int64_t num_blocks, int32_t num_kv_heads, int32_t block_size,
                             int32_t head_dim, int32_t layer_index, const int32_t *block_tables,
                             int32_t block_table_stride, const int32_t *seq_lens,
                             const int32_t *cu_seqlens, int32_t num_seqs, int32_t max_seq_len,
                             void *key_out, void *value_out, int64_t out_token_stride,
                             int64_t out_head_stride, float k_scale, float v_scale,
                             int32_t dtype, tks_stream_t stream);

/* Decode attention over fp8 pools (tks_paged_attention_decode; same workspace size). */
int32_t tks_paged_attention_decode_fp8(
    const void *query, int64_t q_seq_stride, int64_t q_head_stride, const void *key_cache,
    const void *value_cache, int32_t num_layers, int64_t num_blocks, int32_t num_kv_heads,
    int32_t block_size, int32_t head_dim, int32_t layer_index, const int32_t *block_tables,
    int32_t block_table_stride, const int32_t *seq_lens, const int32_t *seq_order,
    int32_t num_seqs, int32_t num_q_heads, int32_t max_seq_len, float scale,
    int32_t pages_per_split, void *out, int64_t out_seq_stride, int64_t out_head_stride,
    void *workspace, int64_t workspace_bytes, float k_scale, float v_scale, int32_t dtype,
    tks_stream_t stream);

/* Chunked-prefill attention over fp8 pools (tks_paged_attention_prefill).
 * For shapes the MFMA prefill kernel serves (bf16/fp16 queries, Dh 64/128,
 * block size a multiple of 16), the pages the batch reads are first decoded
 * into a caller-owned workspace (a dense [num_seqs * block_table_stride] page
 * pool in `dtype` plus its identity block table); its size comes from
 * tks_paged_attention_prefill_fp8_workspace_bytes with the same shapes (0: no
 * workspace needed, the VALU kernel reads the fp8 pool directly). The
 * workspace must be 16-byte aligned; no initial contents are required;
 * launches sharing it must be stream-ordered. */
int64_t tks_paged_attention_prefill_fp8_workspace_bytes(int32_t num_seqs, int32_t num_q_heads,
                                                        int32_t num_kv_heads, int32_t head_dim,
                                                        int32_t block_size,
                                                        int32_t block_table_stride,
                                                        int32_t max_seq_len, int32_t dtype);

int32_t tks_paged_attention_prefill_fp8(
    const void *query, int64_t q_token_stride, int64_t q_head_stride, const void *key_cache,
    const void *value_cache, int32_t num_layers, int64_t num_blocks, int32_t num_kv_heads,
    int32_t block_size, int32_t head_dim, int32_t layer_index, const int32_t *block_tables,
    int32_t block_table_stride, const int32_t *seq_lens, const int32_t *cu_seqlens_q,
    const int32_t *seq_order, int32_t num_seqs, int64_t num_tokens, int32_t num_q_heads,
    int32_t max_query_len, int32_t max_seq_len, float scale, void *out, int64_t out_token_stride,
    int64_t out_head_stride, void *workspace, int64_t workspace_bytes, float k_scale,
    float v_scale, int32_t dtype, tks_stream_t stream);

/* A decode step's RoPE, quantizing KV append and attention in one call
 * (tks_rope_append_paged_decode on fp8 pools): bit-identical to
 * tks_rope_kv_append_fp8 followed by tks_paged_attention_decode_fp8 with the same
 * arguments. */
int32_t tks_rope_append_paged_decode_fp8(
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
    tks_stream_t stream);

/* ------------------------------------------------------------------------
 * fp8 K/V pools with one fp32 scale per pool row (a further variant behind
 * PagedKVStorage, tokserve/engine/paged/storage.py:40-56, where the reference
 * keeps pools in the model dtype). Codes as above in [L, NB, Hkv, BS, Dh];
 * k_scales and v_scales are float [L, NB, Hkv, BS] beside them, one per (token,
 * KV head) slot, written by the appends:
 *   s       = amax / 448, amax = max |x_d| over the row's Dh values (NaN if one
 *             is NaN), and s = 1 where that is 0, NaN or infinite
 *   stored  = e4m3(clamp(x / s, -448, 448))   round to nearest even, NaN kept
 *   decoded = float(stored) * s
 * x is the row in `dtype` (the rotated key row rounded to `dtype` when RoPE is
 * fused in). Every entry takes the arguments of its per-pool-scale counterpart
 * with the two scale arrays in place of k_scale and v_scale; attention computes
 * exactly the function of its counterpart on the decoded pools, in fp32, with
 * each key's scale applied to its scores and each value's to its probabilities.
 * Rows no sequence has written are never read into an output (their codes and
 * scales may hold anything). The decode's fused RoPE + append runs in the
 * attention launch, as its per-pool counterpart does, where the MFMA decode takes
 * the shape (bf16 / fp16 queries, 16-byte aligned new rows): the new rows are
 * quantized with scales of their own, attended to and written with them, bit for
 * bit as tks_rope_kv_append_fp8_rows followed by tks_paged_attention_decode_fp8_rows;
 * elsewhere it runs as those two launches.
 */
int32_t tks_kv_append_fp8_rows(const void *key, int64_t key_token_stride,
                               int64_t key_head_stride, const void *value,
                               int64_t value_token_stride, int64_t value_head_stride,
                               int64_t num_tokens, void *key_cache, void *value_cache,
                               float *k_scales, float *v_scales, int32_t num_layers,
                               int64_t num_blocks, int32_t num_kv_heads, int32_t block_size,
                               int32_t head_dim, int32_t layer_index, const int64_t *slot_mapping,
                               int32_t dtype, tks_stream_t stream);

int32_t tks_paged_gather_fp8_rows(const void *key_cache, const void *value_cache,
                                  const float *k_scales, const float *v_scales, int32_t num_layers,
                                  int64_t num_blocks, int32_t num_kv_heads, int32_t block_size,
                                  int32_t head_dim, int32_t layer_index,
                                  const int32_t *block_tables, int32_t block_table_stride,
                                  const int32_t *seq_lens, const int32_t *cu_seqlens,
                                  int32_t num_seqs, int32_t max_seq_len, void *key_out,
                                  void *value_out, int64_t out_token_stride,
                                  int64_t out_head_stride, int32_t dtype, tks_stream_t stream);

int32_t tks_paged_attention_decode_fp8_rows(
    const void *query, int64_t q_seq_stride, int64_t q_head_stride, const void *key_cache,
    const void *value_cache, const float *k_scales, const float *v_scales, int32_t num_layers,
    int64_t num_blocks, int32_t num_kv_heads, int32_t block_size, int32_t head_dim,
    int32_t layer_index, const int32_t *block_tables, int32_t block_table_stride,
    const int32_t *seq_lens, const int32_t *seq_order, int32_t num_seqs, int32_t num_q_heads,
    int32_t max_seq_len, float scale, int32_t pages_per_split, void *out,
    int64_t out_seq_stride, int64_t out_head_stride, void *workspace, int64_t workspace_bytes,
    int32_t dtype, tks_stream_t stream);

/* The workspace size is tks_paged_attention_prefill_fp8_workspace_bytes'. */
int32_t tks_paged_attention_prefill_fp8_rows(
    const void *query, int64_t q_token_stride, int64_t q_head_stride, const void *key_cache,
    const void *value_cache, const float *k_scales, const float *v_scales, int32_t num_layers,
    int64_t num_blocks, int32_t num_kv_heads, int32_t block_size, int32_t head_dim,
    int32_t layer_index, const int32_t *block_tables, int32_t block_table_stride,
    const int32_t *seq_lens, const int32_t *cu_seqlens_q, const int32_t *seq_order,
    int32_t num_seqs, int64_t num_tokens, int32_t num_q_heads, int32_t max_query_len,
    int32_t max_seq_len, float scale, void *out, int64_t out_token_stride,
    int64_t out_head_stride, void *workspace, int64_t workspace_bytes, int32_t dtype,
    tks_stream_t stream);

int32_t tks_rope_kv_append_fp8_rows(
    const void *query, void *query_out, int64_t q_token_stride, int64_t q_head_stride,
    int64_t qo_token_stride, int64_t qo_head_stride, int32_t num_q_heads, const void *key,
    void *key_out, int64_t k_token_stride, int64_t k_head_stride, int64_t ko_token_stride,
    int64_t ko_head_stride, const void *value, int64_t v_token_stride, int64_t v_head_stride,
    int32_t num_kv_heads, int64_t num_tokens, int32_t head_dim, const int64_t *positions,
    const void *cos_cache, const void *sin_cache, int64_t cache_len, void *key_cache,
    void *value_cache, float *k_scales, float *v_scales, int32_t num_layers, int64_t num_blocks,
    int32_t block_size, int32_t layer_index, const int64_t *slot_mapping, int32_t dtype,
    tks_stream_t stream);

int32_t tks_rope_append_paged_decode_fp8_rows(
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
    int32_t dtype, tks_stream_t stream);

/* ------------------------------------------------------------------------
 * RMSNorm over the last dimension.
 * Replaces triton_rms_norm (tokserve/kernels/rmsnorm.py:6-45, kernel
 * tokserve/kernels/_triton_rmsnorm.py:10-38) and RMSNorm.forward
 * (tokserve/engine/layers.py:29-42):
 *   out = weight * to_input_dtype(x * rsqrt(mean(x^2) + epsilon))
 * reduced in fp32, rounded to input_dtype before the weight multiply, the
 * product rounded once to out_dtype. Valid (input, weight, out) dtype triples
 * follow torch type promotion: weight fp32 -> out fp32; weight == input -> out input.
 * If residual != NULL (fused residual add, tokserve/engine/model.py:73,82):
 *   x = to_input_dtype(input + residual) is written to residual_out first,
 *   then normalised. residual_out may alias input or residual.
 */
int32_t tks_rms_norm(const void *input, int64_t input_row_stride, const void *residual,
                     int64_t residual_row_stride, void *residual_out,
                     int64_t residual_out_row_stride, const void *weight, void *out,
                     int64_t out_row_stride, int64_t num_rows, int32_t hidden_size,
                     float epsilon, int32_t input_dtype, int32_t weight_dtype,
                     int32_t out_dtype, tks_stream_t stream);

/* ------------------------------------------------------------------------
 * Rotary position embedding (half rotation) on Q and K in one launch.
 * Replaces triton_apply_rope (tokserve/kernels/rope.py:8-63, kernel
 * tokserve/kernels/_triton_rope.py:10-68) and apply_rope (tokserve/engine/rope.py:106-153):
 *   out[d] = r(x[d]*cos[p][d]) + r(rot(x)[d]*sin[p][d]),  rot(x) = cat(-x2, x1)
 * with each product rounded to dtype before the add (r = round to dtype).
 * Element (b, h, t, d) of Q lives at q[b*q_sb + h*q_sh + t*q_st + d] and is
 * written to q_out[b*qo_sb + h*qo_sh + t*qo_st + d] (q_out may equal q).
 * Same for K with num_kv_heads. Position of token t: positions[t] (int64).
 * cos_cache / sin_cache: [cache_len, head_dim/2] in dtype, row p holding
 * cos/sin(fp32(p) * inv_freq) cast to dtype (tokserve/engine/rope.py:28-87).
 * Positions outside [0, cache_len) are clamped; callers validate them.
 */
int32_t tks_rope(const void *query, void *query_out, int64_t q_sb, int64_t q_sh, int64_t q_st,
                 int64_t qo_sb, int64_t qo_sh, int64_t qo_st, int32_t num_q_heads,
                 const void *key, void *key_out, int64_t k_sb, int64_t k_sh, int64_t k_st,
                 int64_t ko_sb, int64_t ko_sh, int64_t ko_st, int32_t num_kv_heads,
                 int32_t batch, int64_t num_tokens, int32_t head_dim, const int64_t *positions,
                 const void *cos_cache, const void *sin_cache, int64_t cache_len, int32_t dtype,
                 tks_stream_t stream);

/* ------------------------------------------------------------------------
 * RoPE fused with the KV append, for a packed step (one launch where the model
 * layer would run tks_rope and then tks_kv_append; the reference does the two
 * in turn per request, tokserve/engine/attention.py:247-265 and
 * tokserve/engine/paged/sequence_cache.py:86-131):
 *   query token t, head h (strides q_ts, q_hs) is rotated at positions[t] into
 *   query_out (may equal query); key rows are rotated and written to pool slot
 *   slot_mapping[t] of layer_index (and to key_out when it is not NULL); value
 *   rows are copied to the same slot. Pools [L, NB, Hkv, BS, Dh] in `dtype`.
 * Results are bit-identical to tks_rope followed by tks_kv_append of the rotated
 * keys; negative slots skip the token's append (its Q is still rotated).
 */
int32_t tks_rope_kv_append(const void *query, void *query_out, int64_t q_ts, int64_t q_hs,
                           int64_t qo_ts, int64_t qo_hs, int32_t num_q_heads, const void *key,
                           void *key_out, int64_t k_ts, int64_t k_hs, int64_t ko_ts,
                           int64_t ko_hs, const void *value, int64_t v_ts, int64_t v_hs,
                           int32_t num_kv_heads, int64_t num_tokens, int32_t head_dim,
                           const int64_t *positions, const void *cos_cache,
                           const void *sin_cache, int64_t cache_len, void *key_cache,
                           void *value_cache, int32_t num_layers, int64_t num_blocks,
                           int32_t block_size, int32_t layer_index,
                           const int64_t *slot_mapping, int32_t dtype, tks_stream_t stream);

/* tks_rope_kv_append on fp8 pools (the e4m3 pool variant described with
 * tks_kv_append_fp8): the rotated key row, held at `dtype` precision, and the value
 * row are written as e4m3(clamp(x / scale)) with k_scale / v_scale. Bit-identical to
 * tks_rope followed by tks_kv_append_fp8 of the rotated keys.
 */
int32_t tks_rope_kv_append_fp8(const void *query, void *query_out, int64_t q_ts, int64_t q_hs,
                               int64_t qo_ts, int64_t qo_hs, int32_t num_q_heads,
                               const void *key, void *key_out, int64_t k_ts, int64_t k_hs,
                               int64_t ko_ts, int64_t ko_hs, const void *value, int64_t v_ts,
                               int64_t v_hs, int32_t num_kv_heads, int64_t num_tokens,
                               int32_t head_dim, const int64_t *positions,
                               const void *cos_cache, const void *sin_cache, int64_t cache_len,
                               void *key_cache, void *value_cache, int32_t num_layers,
                               int64_t num_blocks, int32_t block_size, int32_t layer_index,
                               const int64_t *slot_mapping, float k_scale, float v_scale,
                               int32_t dtype, tks_stream_t stream);

/* ------------------------------------------------------------------------
 * Greedy token selection: first index of the row maximum (NaN counts as the
 * maximum, as torch.argmax does).
 * Replaces select_greedy (tokserve/generation/greedy.py:6-18) on a (B, V) batch.
 * logits[r*row_stride + v]; out_ids[r] (int64).
 */
int32_t tks_argmax(const void *logits, int64_t row_stride, int64_t num_rows, int64_t vocab_size,
                   int64_t *out_ids, int32_t dtype, tks_stream_t stream);

/* ------------------------------------------------------------------------
 * SwiGLU activation on fused gate/up rows: for each row r and j < I,
 *   out[r*out_row_stride + j] = r(r(silu(g)) * u),  g = gate_up[r*gate_up_row_stride + j],
 *   u = gate_up[r*gate_up_row_stride + I + j],  silu(g) = g / (1 + exp(-g)) in fp32,
 * r = rounding to dtype. Replaces `functional.silu(gate_proj(x)) * up_proj(x)` of
 * SwiGLU.forward (tokserve/engine/layers.py:84-91) after one GEMM over the stacked
 * gate/up weights.
 */
int32_t tks_silu_mul(const void *gate_up, int64_t gate_up_row_stride, int64_t num_rows,
                     int64_t intermediate_size, void *out, int64_t out_row_stride, int32_t dtype,
                     tks_stream_t stream);

/* ------------------------------------------------------------------------
 * Elementwise out[i] = x[i] + y[i] over num_elements contiguous elements.
 * Replaces vector_add (tokserve/kernels/vector.py:6-41). dtype FLOAT32 or
 * FLOAT16 (TKS_ERR_TYPE otherwise); num_elements == 0 launches nothing.
 */
int32_t tks_vector_add(const void *x, const void *y, void *out, int64_t num_elements, int32_t dtype,
                       tks_stream_t stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* TOKSERVE_HIP_H */
