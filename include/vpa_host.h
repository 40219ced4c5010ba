/*
 * vpa_host.h — host-side bookkeeping of the paged KV cache: pool sizing, the
 * block manager, the per-step metadata builders and the decode-graph padding
 * rules. These restate vasr-paged-attn's Rust host code
 * (paged_cache_runtime.rs, paged_kv_cache.rs, cuda_graph.rs) so that a C or
 * C++ caller gets the same metadata the paged kernels of vpa.h expect.
 *
 * Conventions: plain host pointers and sizes; int status codes of vpa.h
 * (VPA_OK, VPA_ERR_INVALID_ARGUMENT, VPA_ERR_CAPACITY, VPA_ERR_NOT_FOUND)
 * with the message in vpa_last_error(). No function touches device memory.
 * A block manager is not thread-safe (the reference guards its runtime with
 * a mutex, paged_cache_runtime.rs:707).
 *
 * Ragged block tables are passed as a 2-D uint32 array with row stride
 * `stride` and per-row lengths `table_lens`.
 */
#ifndef VPA_HOST_H_
#define VPA_HOST_H_

#include <stddef.h>
#include <stdint.h>

#include "vpa.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- sizing */

/* KV bytes of one block over all layers: layers * kv_heads * head_dim *
 * block_size * 2 * sizeof(dtype). bytes_per_paged_block,
 * paged_cache_runtime.rs:46-72. */
int vpa_bytes_per_paged_block(int32_t num_layers, int32_t num_kv_heads, int32_t head_dim,
                              int32_t block_size, int32_t dtype, uint64_t* bytes);

/* Pool blocks for a token capacity: ceil(tokens / block_size) + 1 (block 0
 * is the null block). PagedCacheMemory::ContextSize,
 * paged_cache_runtime.rs:161. */
int vpa_pool_blocks_for_context(int64_t tokens, int32_t block_size, int64_t* num_blocks);

/* Pool blocks for a byte budget: budget / bytes_per_block + 1; fails when
 * that is <= 1. blocks_for_byte_budget, paged_cache_runtime.rs:74-87. */
int vpa_pool_blocks_for_byte_budget(uint64_t byte_budget, uint64_t bytes_per_block,
                                    int64_t* num_blocks);

/* Pool blocks for `fraction` of the current device's memory: budget =
 * floor(total_MiB * fraction) - used_MiB (in MiB, from hipMemGetInfo), then
 * vpa_pool_blocks_for_byte_budget. PagedCacheMemory::GpuMemoryFraction
 * (paged_cache_runtime.rs:136-150, which reads nvidia-smi). The library's
 * device code is loaded on the current device before the free memory is
 * read, so used_MiB already counts the static decode scratch of
 * vpa_paged_attention_noalloc (64 MiB per GPU by default, build-time
 * VPA_NOALLOC_SCRATCH_MIB), which every process that loads the library holds
 * on each GPU it runs on. */
int vpa_pool_blocks_for_memory_fraction(float fraction, uint64_t bytes_per_block,
                                        int64_t* num_blocks);

/* --------------------------------------------------------- block manager */

/* FIFO free list over block ids 1..num_blocks-1 (block 0 is reserved for
 * padded batches); per-request block lists. PagedBlockManager,
 * paged_cache_runtime.rs:217-380. */
typedef struct vpa_block_manager vpa_block_manager;

int vpa_block_manager_create(int64_t num_blocks, int32_t block_size, vpa_block_manager** out);
void vpa_block_manager_destroy(vpa_block_manager* manager);
int64_t vpa_block_manager_free_blocks(const vpa_block_manager* manager);
int64_t vpa_block_manager_blocks_for_request(const vpa_block_manager* manager,
                                             uint64_t request_id);
int64_t vpa_block_manager_total_allocated_blocks(const vpa_block_manager* manager);
/* 1 if the request can grow to num_tokens tokens, else 0. */
int vpa_block_manager_slots_available(const vpa_block_manager* manager, uint64_t request_id,
                                      int64_t num_tokens);
/* Grow the request to cover num_tokens tokens, taking blocks from the front
 * of the free list; *allocated = 0 (and nothing changes) when the pool is
 * short. try_allocate_slots, :286-318. */
int vpa_block_manager_try_allocate(vpa_block_manager* manager, uint64_t request_id,
                                   int64_t num_tokens, int32_t* allocated);
/* As try_allocate, but a full pool is VPA_ERR_CAPACITY. allocate_slots, :275-284. */
int vpa_block_manager_allocate(vpa_block_manager* manager, uint64_t request_id,
                               int64_t num_tokens);
/* Shrink to ceil(num_tokens / block_size) blocks; the tail goes back to the
 * end of the free list in reverse order. trim_request_to_num_tokens, :320-335. */
int vpa_block_manager_trim(vpa_block_manager* manager, uint64_t request_id, int64_t num_tokens);
/* Release every block of the request (reverse order, to the end of the free
 * list); unknown ids are ignored. free_request, :348-357. */
int vpa_block_manager_free_request(vpa_block_manager* manager, uint64_t request_id);
/* Copy the request's block ids; VPA_ERR_NOT_FOUND if it has none,
 * VPA_ERR_CAPACITY if `capacity` is too small (count is set either way). */
int vpa_block_manager_block_ids(const vpa_block_manager* manager, uint64_t request_id,
                                uint32_t* ids, int64_t capacity, int64_t* count);
/* Block tables of several requests as a zero-padded [num_requests, cols]
 * array plus the true lengths. block_tables_for, :365-379. */
int vpa_block_manager_block_tables(const vpa_block_manager* manager, const uint64_t* request_ids,
                                   int32_t num_requests, int32_t cols, uint32_t* tables,
                                   int32_t* table_lens);

/* ------------------------------------------------------ metadata builders */

/* Outputs of a metadata builder; the caller owns every array. */
typedef struct vpa_paged_metadata {
  int64_t* slot_mapping;   /* [num_tokens] */
  uint32_t* block_tables;  /* [batch, cols], rows zero-padded */
  uint32_t* context_lens;  /* [batch] */
  uint32_t* cu_seqlens_q;  /* [batch + 1], may be NULL */
  uint32_t* cu_seqlens_kv; /* [batch + 1], may be NULL */
  int32_t cols;            /* in: width of block_tables (>= the longest table) */
  int64_t num_tokens;      /* out: slots written */
  int64_t max_context_len; /* out */
  int64_t max_query_len;   /* out */
  int64_t max_kv_len;      /* out */
  int32_t causal_only;     /* out: prefill_causal_only */
} vpa_paged_metadata;

/* slot = table[position / block_size] * block_size + position % block_size;
 * a missing entry or a block id >= num_blocks is an error.
 * slot_for_block_table_position, paged_kv_cache.rs:74-103. */
int vpa_slot_for_block_table_position(const uint32_t* table, int32_t table_len,
                                      int32_t block_size, int64_t num_blocks, int64_t position,
                                      int64_t* slot);

/* cu[0] = 0, cu[i+1] = cu[i] + lengths[i], in u32 (overflow is an error).
 * cumulative_seqlens_from_lengths, paged_kv_cache.rs:58-72. */
int vpa_cumulative_seqlens(const int64_t* lengths, int32_t n, uint32_t* cu);

/* len tokens per sequence from starts[s]; context_lens given.
 * input_metadata_from_block_tables, paged_kv_cache.rs:547-649. */
int vpa_metadata_from_block_tables(const uint32_t* tables, int32_t stride,
                                   const int32_t* table_lens, int32_t batch,
                                   const int64_t* starts, int32_t len,
                                   const int64_t* context_lens, int32_t block_size,
                                   int64_t num_blocks, vpa_paged_metadata* out);

/* Right-padded prompts: mask 0 gives PAD_SLOT_ID (-1); each sequence's
 * context (and query) length is its count of ones.
 * input_metadata_from_attention_masks, paged_kv_cache.rs:651-773. */
int vpa_metadata_from_attention_masks(const uint32_t* tables, int32_t stride,
                                      const int32_t* table_lens, int32_t batch,
                                      const uint32_t* masks, int32_t seq_len, int32_t block_size,
                                      int64_t num_blocks, vpa_paged_metadata* out);

/* Packed prefill: sequence s contributes query_lens[s] (> 0) tokens at
 * positions 0..; context = query length.
 * input_metadata_from_query_lens, paged_kv_cache.rs:775-869. */
int vpa_metadata_from_query_lens(const uint32_t* tables, int32_t stride,
                                 const int32_t* table_lens, int32_t batch,
                                 const int64_t* query_lens, int32_t block_size,
                                 int64_t num_blocks, vpa_paged_metadata* out);

/* Decode steps 0..steps-1 of a batch: step t of sequence s writes position
 * prompt_lens[s] + t (slot through its table) with context position + 1.
 * slots/contexts are [steps, batch], max_context_lens [steps]; the block
 * tables are zero-padded to `cols`, which must be at least the longest
 * table, or exactly vpa_bucket_block_table_cols(longest) when graph_buckets
 * is non-zero (the cuda-graph build). A context above
 * max_tokens_per_sequence is an error.
 * decode_metadata_for_batch_steps, paged_kv_cache.rs:924-1044. */
int vpa_decode_metadata_for_batch_steps(const uint32_t* tables, int32_t stride,
                                        const int32_t* table_lens, int32_t batch,
                                        const int64_t* prompt_lens, int32_t steps,
                                        int32_t block_size, int64_t num_blocks,
                                        int64_t max_tokens_per_sequence, int32_t graph_buckets,
                                        int32_t cols, int64_t* slots, uint32_t* context_lens,
                                        int64_t* max_context_lens, uint32_t* block_tables);

/* Slot of a sequence of a contiguous (new_batched) cache:
 * sequence * blocks_per_sequence * block_size + position.
 * slot_for_sequence_position, paged_kv_cache.rs:356-378. */
int vpa_contiguous_slot(int64_t sequence, int64_t position, int64_t batch,
                        int64_t blocks_per_sequence, int32_t block_size,
                        int64_t max_tokens_per_sequence, int64_t* slot);

/* -------------------------------------------------- decode-graph padding */

/* Batch bucket a graph is captured for: 1, 2, 4, 8, then multiples of 16,
 * capped at max_batch; 0 when actual is 0 or above max_batch.
 * cuda_graph_batch_bucket, cuda_graph.rs:28-40. */
int32_t vpa_graph_batch_bucket(int32_t actual_batch, int32_t max_batch);

/* All buckets up to min(max_batch, 256), max_batch included.
 * cuda_graph_batch_buckets, cuda_graph.rs:42-61. */
int vpa_graph_batch_buckets(int32_t max_batch, int32_t* buckets, int32_t capacity,
                            int32_t* count);

/* Block-table width of a graph: next power of two of `blocks`, at least
 * ceil(256 / block_size). bucket_block_table_cols, cuda_graph.rs:68-75. */
int64_t vpa_bucket_block_table_cols(int64_t blocks, int32_t block_size);

/* Pad a decode batch's metadata to max_batch rows and cols_out columns:
 * padded rows get slot 0, context 1 and an all-zero table; columns are
 * padded by repeating each row's last column (zeros for a 0-wide table).
 * input_ids may be NULL; padded ids are 0.
 * pad_decode_batch_to_max + pad_metadata_block_tables, cuda_graph.rs:373-486. */
int vpa_pad_decode_batch(int32_t max_batch, int32_t actual_batch, const uint32_t* input_ids,
                         const int64_t* slots, const uint32_t* context_lens,
                         const uint32_t* block_tables, int32_t cols_in, int32_t cols_out,
                         uint32_t* out_input_ids, int64_t* out_slots,
                         uint32_t* out_context_lens, uint32_t* out_block_tables);

#ifdef __cplusplus
}
#endif

#endif /* VPA_HOST_H_ */
