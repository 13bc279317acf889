/*
 * kvslots.c -- TEST INFRASTRUCTURE ONLY (the oracle's integer/byte work).
 *
 * Plain-C restatement of tokserve's paged-KV addressing and copies:
 *   slot of logical position p   tokserve/engine/paged/block_table.py:53-67
 *     block = block_ids[p / BS], offset = p % BS, slot = block * BS + offset
 *   KV append (write_token)      tokserve/engine/paged/storage.py:64-89,
 *                                tokserve/engine/paged/sequence_cache.py:120-129
 *     pool[layer, block, h, offset, :] = row[h, :]
 *   block-table gather           tokserve/engine/paged/sequence_cache.py:157-193,
 *                                tokserve/engine/paged/storage.py:103-116
 * Element-type agnostic: rows are copied as bytes, so results are bit-exact.
 * Pools are [L, NB, Hkv, BS, Dh] contiguous; strides are in elements.
 */
#include <stdint.h>
#include <string.h>

/* Slot of logical position `position` through a block table, or -1 when the
 * position is beyond the table (the reference raises IndexError there). */
int64_t oracle_slot(const int32_t *block_ids, int64_t num_ids, int32_t block_size,
                    int64_t position) {
  if (position < 0 || block_size <= 0) return -1;
  const int64_t logical = position / block_size;
  if (logical >= num_ids) return -1;
  return (int64_t)block_ids[logical] * block_size + position % block_size;
}

/* slot_mapping for a ragged batch: sequence b appends new_lens[b] tokens
 * starting at position start[b]; its table is row b of block_tables. */
int32_t oracle_slot_mapping(const int32_t *block_tables, int32_t table_stride,
                            const int64_t *start, const int64_t *new_lens, int32_t num_seqs,
                            int32_t block_size, int64_t *slots_out) {
  int64_t n = 0;
  for (int32_t b = 0; b < num_seqs; ++b) {
    for (int64_t i = 0; i < new_lens[b]; ++i) {
      const int64_t s =
          oracle_slot(block_tables + (int64_t)b * table_stride, table_stride, block_size, start[b] + i);
      if (s < 0) return -1;
      slots_out[n++] = s;
    }
  }
  return 0;
}

static int64_t pool_offset(int64_t num_blocks, int32_t num_kv_heads, int32_t block_size,
                           int32_t head_dim, int32_t layer, int64_t block, int32_t head,
                           int64_t offset) {
  return ((((int64_t)layer * num_blocks + block) * num_kv_heads + head) * block_size + offset) *
         head_dim;
}

/* Write rows key[t, h, :] (strides in elements) to the slots; negative slots skip. */
int32_t oracle_kv_append(const void *key, int64_t k_ts, int64_t k_hs, const void *value,
                         int64_t v_ts, int64_t v_hs, int64_t num_tokens, void *key_cache,
                         void *value_cache, int64_t num_blocks, int32_t num_kv_heads,
                         int32_t block_size, int32_t head_dim, int32_t layer,
                         const int64_t *slots, int32_t elem_size) {
  const size_t row = (size_t)head_dim * (size_t)elem_size;
  for (int64_t t = 0; t < num_tokens; ++t) {
    const int64_t slot = slots[t];
    if (slot < 0) continue;
    if (slot >= num_blocks * block_size) return -1;
    const int64_t block = slot / block_size, offset = slot % block_size;
    for (int32_t h = 0; h < num_kv_heads; ++h) {
      const int64_t dst =
          pool_offset(num_blocks, num_kv_heads, block_size, head_dim, layer, block, h, offset);
      memcpy((char *)key_cache + dst * elem_size,
             (const char *)key + (t * k_ts + h * k_hs) * elem_size, row);
      memcpy((char *)value_cache + dst * elem_size,
             (const char *)value + (t * v_ts + h * v_hs) * elem_size, row);
    }
  }
  return 0;
}

/* Gather each sequence's first seq_lens[b] positions into out[(cu[b] + p), h, :]. */
int32_t oracle_paged_gather(const void *key_cache, const void *value_cache, int64_t num_blocks,
                            int32_t num_kv_heads, int32_t block_size, int32_t head_dim,
                            int32_t layer, const int32_t *block_tables, int32_t table_stride,
                            const int32_t *seq_lens, const int32_t *cu, int32_t num_seqs,
                            void *key_out, void *value_out, int64_t o_ts, int64_t o_hs,
                            int32_t elem_size) {
  const size_t row = (size_t)head_dim * (size_t)elem_size;
  for (int32_t b = 0; b < num_seqs; ++b) {
    const int32_t *table = block_tables + (int64_t)b * table_stride;
    for (int64_t p = 0; p < seq_lens[b]; ++p) {
      const int64_t slot = oracle_slot(table, table_stride, block_size, p);
      if (slot < 0 || slot >= num_blocks * block_size) return -1;
      const int64_t block = slot / block_size, offset = slot % block_size;
      for (int32_t h = 0; h < num_kv_heads; ++h) {
        const int64_t src =
            pool_offset(num_blocks, num_kv_heads, block_size, head_dim, layer, block, h, offset);
        const int64_t dst = (cu[b] + p) * o_ts + h * o_hs;
        memcpy((char *)key_out + dst * elem_size, (const char *)key_cache + src * elem_size, row);
        memcpy((char *)value_out + dst * elem_size, (const char *)value_cache + src * elem_size,
               row);
      }
    }
  }
  return 0;
}
