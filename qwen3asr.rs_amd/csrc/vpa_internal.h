// Host-side internals shared by the C-ABI layer and the kernel launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/vpa.h"

namespace vpa {

// Thread-local error message; returns `code` for tail calls.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Geometry of one layer's paged cache (both K and V tiles are
// head_dim*block_size contiguous elements per (block, head)).
struct CacheGeom {
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t block_size;
  int64_t num_blocks;
  int64_t block_stride;  // elements
  int64_t head_stride;   // elements
  // decode only: num_kv_heads counts kv_rep replicas of every cache head
  // (head j reads cache head j / kv_rep), for more query heads per kv head
  // than a kernel instance serves
  int32_t kv_rep = 1;
};

// Decode split-K partition length in tokens of the generic decode kernel (a
// multiple of every supported block size).
constexpr int kDecodePartitionTokens = 256;
// Smallest partition length any decode kernel uses; sizes the workspace.
constexpr int kDecodeMinPartitionTokens = 128;
// Upper bound on split-K partitions per sequence handled by the reduce kernel.
constexpr int kDecodeMaxPartitions = 2048;

// Caller workspace of paged_attention, carved in this order (each piece
// 256-byte aligned):
struct DecodeWorkspace {
  float* part_out;   // [num_seqs, num_heads, max_parts, head_dim] split-K partials
  float* part_max;   // [num_seqs, num_heads, max_parts]
  float* part_sum;   // [num_seqs, num_heads, max_parts]
  uint2* items;      // [num_seqs * max(1, max_parts)] work list {seq << 16 | partition, length}
  uint32_t* queue;   // [2]: next work unit, number of items
  int max_parts;     // ceil(max_context_len / partition tokens of the layout)
  bool planned = false;  // the work list is already in the workspace (skip the plan launch)
};

// New K/V rows of a decode step appended by the decode launch itself
// (vpa_reshape_and_cache_paged_attention): row s (one token, num_kv_heads *
// head_dim elements of the cache type) goes to position context_lens[s] - 1
// of sequence s's block table.
struct DecodeAppend {
  const void* key;
  const void* value;
  int64_t key_token_stride;
  int64_t value_token_stride;
};

// Largest batch whose decode append runs inside the decode launch (the
// environment variable VPA_FUSED_APPEND_MAX_SEQS, read once, overrides it).
constexpr int kFusedAppendMaxSeqs = 48;
// True when vpa_reshape_and_cache_paged_attention runs its append inside the
// decode launch (16-bit cache of the query's type on the rows kernel with a
// (block, head) tile of at least 2 KiB, at most kFusedAppendMaxSeqs sequences).
bool decode_fuses_append(int dtype, int cache_dtype, int head_dim, int block_size,
                         int num_seqs, int group);
// Query heads per kv head a decode kernel instance serves for G query heads
// per kv head (4, 2 or 1, dividing G); larger G runs G / that replicas.
int decode_kernel_group(int group);

// Compute units of the current device (cached per device).
int device_cu_count();

// The library's own decode scratch (the allocation-free entry point): its
// size and the lookup of its address on the current device.
struct DecodeScratch {
  size_t bytes;
  int (*address)(const char* op, void** out);
  // Called after every argument check, right before the call's launches on
  // `stream` (VPA_OK or an error status, then nothing is launched), and
  // after them with their status (returns the call's status).
  int (*before)(const char* op, void* stream);
  int (*after)(const char* op, void* stream, int rc);
};

// Bytes of the static decode scratch on each GPU (VPA_NOALLOC_SCRATCH_MIB).
size_t noalloc_scratch_bytes();
// Loads this library's device code object on the current device (the HIP
// runtime loads it lazily, and with it reserves the static decode scratch)
// by looking up the scratch's address; VPA_OK or a HIP error status.
int load_device_code(const char* op);

// vpa_paged_attention and its variants: every argument check, then the
// launches. With `scratch` the workspace arguments are ignored: after the
// checks the call takes the library's scratch, laid out for the kernel that
// runs (decode_part_tokens), and fails with VPA_ERR_WORKSPACE when that
// layout does not fit it.
int paged_attention_impl(void* out, const void* query, const float* k_scale,
                         const float* v_scale, const void* key_cache, const void* value_cache,
                         const uint32_t* block_tables, int32_t block_table_stride,
                         const uint32_t* context_lens, const float* alibi_slopes,
                         int32_t max_context_len, float softmax_scale, float softcapping,
                         const float* sinks, int32_t num_seqs, int32_t num_heads,
                         int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                         int64_t num_blocks, int64_t cache_block_stride,
                         int64_t cache_head_stride, int32_t dtype, int32_t cache_dtype,
                         void* workspace, size_t workspace_bytes, void* stream, bool planned,
                         const DecodeScratch* scratch, const char* op,
                         const DecodeAppend* append = nullptr);

// Split-K partition (tokens) of the decode kernel that runs for a query
// dtype and head_dim: the rows kernel's chunk, or the generic kernel's
// partition.
int decode_part_tokens(int dtype, int head_dim, int block_size);
// Decode scratch bytes and layout for partitions of part_tokens tokens; the
// caller workspace of vpa_paged_attention uses kDecodeMinPartitionTokens
// (valid for every kernel), the library's own scratch the running kernel's
// partition (decode_part_tokens).
size_t decode_workspace_bytes(int num_seqs, int num_heads, int head_dim, int max_context_len,
                              int part_tokens = kDecodeMinPartitionTokens);
DecodeWorkspace carve_decode_workspace(void* base, int num_seqs, int num_heads, int head_dim,
                                       int max_context_len,
                                       int part_tokens = kDecodeMinPartitionTokens);

// Launchers return hipSuccess or the launch error. Arguments are validated by
// the caller.
// cache_dtype is dtype (bit-exact copy) or VPA_DTYPE_FP8_E4M3 (quantised
// with the device scalars *k_scale / *v_scale).
hipError_t launch_reshape_and_cache(int dtype, int cache_dtype, const void* key,
                                    const void* value, int64_t key_token_stride,
                                    int64_t value_token_stride, void* key_cache,
                                    void* value_cache, const int64_t* slot_mapping,
                                    int64_t num_tokens, const CacheGeom& g, const float* k_scale,
                                    const float* v_scale, hipStream_t stream);

// The slot of row t of an append derived from the decode metadata: position
// context_lens[t] - 1 of block-table row t (no slot for an empty context or
// one above cap = min(max_context_len, block_table_stride * block_size)).
struct LastSlots {
  const uint32_t* block_tables = nullptr;
  const uint32_t* context_lens = nullptr;
  int32_t stride = 0;
  int32_t cap = 0;
};
// reshape_and_cache of num_seqs rows, row s at sequence s's last position.
hipError_t launch_append_last_positions(int dtype, int cache_dtype, const void* key,
                                        const void* value, int64_t key_token_stride,
                                        int64_t value_token_stride, void* key_cache,
                                        void* value_cache, const LastSlots& last,
                                        int32_t num_seqs, const CacheGeom& g,
                                        const float* k_scale, const float* v_scale,
                                        hipStream_t stream);

// out_dtype is cache_dtype (copy) or, for an fp8 cache, f32 / f16 / bf16
// (dequantised with *k_scale / *v_scale).
hipError_t launch_gather_kv_cache(int cache_dtype, int out_dtype, void* out_key,
                                  void* out_value, const void* key_cache,
                                  const void* value_cache, const uint32_t* block_tables,
                                  int32_t block_table_stride, const uint32_t* cu_seqlens,
                                  int32_t num_seqs, const CacheGeom& g, const float* k_scale,
                                  const float* v_scale, hipStream_t stream);

// cache_dtype is dtype, or VPA_DTYPE_FP8_E4M3 with a bf16 / f16 query
// (scales are device pointers, read only for fp8).
hipError_t launch_paged_decode(int dtype, int cache_dtype, void* out, const void* query,
                               const void* key_cache, const void* value_cache,
                               const uint32_t* block_tables, int32_t block_table_stride,
                               const uint32_t* context_lens, int32_t max_context_len,
                               float scale, const float* k_scale, const float* v_scale,
                               int32_t num_seqs, int32_t num_heads, const CacheGeom& g,
                               const DecodeWorkspace& ws, hipStream_t stream,
                               const DecodeAppend* append = nullptr);

hipError_t launch_prefill_paged(int dtype, int cache_dtype, void* out, const void* query,
                                const void* key_cache, const void* value_cache,
                                const uint32_t* block_tables, int32_t block_table_stride,
                                const uint32_t* cu_seqlens_q, const uint32_t* context_lens,
                                int32_t num_seqs, int32_t max_query_len, int32_t max_kv_len,
                                int64_t total_query_rows, float scale, float denom_eps,
                                int32_t causal, int32_t num_heads, const CacheGeom& g,
                                const float* k_scale, const float* v_scale,
                                hipStream_t stream);

// The vector-ALU prefill (prefill_vector_kernels.hip): f32 queries over f32
// or fp8 caches, any number of query heads per kv head, and the 16-bit
// shapes the MFMA kernel does not take; also the decode of the head-dim /
// block-size pairs no decode kernel takes (cu_seqlens_q null: one query per
// sequence). Same arguments as launch_prefill_paged.
bool prefill_vector_supported(int dtype, int cache_dtype, int head_dim, int block_size);
int64_t prefill_vector_workgroups(int32_t num_seqs, int32_t max_query_len, int32_t group,
                                  int32_t num_kv_heads);
hipError_t launch_prefill_vector(int dtype, int cache_dtype, void* out, const void* query,
                                 const void* key_cache, const void* value_cache,
                                 const uint32_t* block_tables, int32_t block_table_stride,
                                 const uint32_t* cu_seqlens_q, const uint32_t* context_lens,
                                 int32_t num_seqs, int32_t max_query_len, int32_t max_kv_len,
                                 int64_t total_query_rows, float scale, float denom_eps,
                                 int32_t causal, int32_t num_heads, const CacheGeom& g,
                                 const float* k_scale, const float* v_scale,
                                 hipStream_t stream);

// Query positions one prefill workgroup covers for a GQA group size.
int prefill_positions_per_workgroup(int group);
// True when the MFMA prefill kernel is compiled for this combination.
bool prefill_supported(int dtype, int cache_dtype, int head_dim, int block_size, int group);

// Builds the decode work list into the workspace (the plan launch of
// launch_paged_decode on its own); a no-op for configurations whose decode
// kernel takes no work list.
hipError_t launch_decode_plan(int dtype, const uint32_t* context_lens, int32_t max_context_len,
                              int32_t block_table_stride, int32_t num_seqs, const CacheGeom& g,
                              const DecodeWorkspace& ws, hipStream_t stream);

// Next-token ids of `num_rows` logits rows (first maximum, NaN-aware as
// candle's argmax) and the step-start EOS bookkeeping of the decode loop.
hipError_t launch_argmax_rows(int dtype, const void* logits, int64_t row_stride, int32_t vocab,
                              int32_t num_rows, uint32_t* out, hipStream_t stream);
hipError_t launch_consume_tokens(const uint32_t* next_ids, uint8_t* finished,
                                 const int64_t* prev_slot_mapping, uint32_t* generated, uint32_t* gen_len, int32_t gen_capacity,
                                 const uint32_t* eos_ids, int32_t num_eos, uint32_t eos_fill_id,
                                 uint32_t* input_ids, uint32_t* active_count, int32_t num_rows,
                                 hipStream_t stream);

// Device-resident KV block allocation and decode-step metadata.
hipError_t launch_allocate_rows(uint32_t* block_tables, int32_t cols, uint32_t* row_blocks,
                                const uint32_t* target_tokens, uint8_t* ok, uint32_t* ring,
                                uint32_t* ring_state, int32_t ring_cap, int32_t block_size,
                                int32_t num_rows, hipStream_t stream);
hipError_t launch_decode_step_metadata(uint32_t* block_tables, int32_t cols,
                                       uint32_t* row_blocks, uint32_t* positions,
                                       const uint8_t* finished, uint32_t* ring,
                                       uint32_t* ring_state, int32_t ring_cap,
                                       int32_t block_size, int64_t* slot_mapping,
                                       uint32_t* context_lens, uint32_t* status,
                                       int32_t num_rows, hipStream_t stream);
hipError_t launch_release_blocks(const uint32_t* block_tables, int32_t cols,
                                 uint32_t* row_blocks, const uint32_t* keep_blocks,
                                 uint32_t* ring, uint32_t* ring_state, int32_t ring_cap,
                                 int32_t num_rows, hipStream_t stream);

// The decode's read pattern with no compute (vpa_paged_cache_read): 16-bit
// or fp8 caches, head_dim <= 128, tiles of a whole number of KiB (<= 8).
bool paged_read_supported(int cache_dtype, int head_dim, int block_size);
hipError_t launch_paged_read(int cache_dtype, const void* key_cache, const void* value_cache,
                             const uint32_t* block_tables, int32_t block_table_stride,
                             int32_t max_context_len, int32_t num_seqs, const CacheGeom& g,
                             const DecodeWorkspace& ws, uint32_t magic, uint32_t* sink,
                             hipStream_t stream);

// True when a decode kernel is compiled for this (dtype, head_dim, block_size,
// query heads per kv head) combination.
bool decode_supported(int dtype, int head_dim, int block_size, int group);
// 16-bit queries decode with the rows kernel (and its work list) where a
// 16-bit (block, head) tile is 1 to 8 whole KiB (head dims 64 and 128, 96
// at 16- and 32-token blocks, 192 and 256 at 8 and 16); f32 and the other
// shapes with the generic split-K kernel. The work list depends on this
// choice only, so it is the same for every cache type.
bool decode_uses_rows_kernel(int dtype, int head_dim, int block_size);
// fp8 caches under 16-bit queries: on the rows kernel head dims 64 and 128
// at 16- and 32-token blocks, 128 at 8, 96 at 32, 192 at 16, 256 at 8 and
// 16; on the generic split-K kernel 192 and 256 at 32.
bool decode_fp8_shape(int head_dim, int block_size);
// fp8 caches under f32 queries decode on the generic split-K kernel: blocks
// of 16 or 32 tokens with a whole number of 1 KiB wave loads per tile.
bool decode_f32_fp8_shape(int head_dim, int block_size);
bool cache_kernels_supported(int dtype, int head_dim, int block_size);

}  // namespace vpa
