/*
 * vpa.h — C ABI of the MI355X (gfx950) paged-KV hot path for the Qwen3-ASR
 * text decoder.
 *
 * The entry points replace the three Candle ops that vASR imports from the
 * external crate `mistralrs-paged-attn` (re-exported at
 * vasr-paged-attn/src/lib.rs:20-21) plus the paged chunked-prefill attention,
 * keeping the reference's cache layouts and metadata semantics:
 *
 *   key_cache   [num_blocks, num_kv_heads, head_dim / x, block_size, x]
 *   value_cache [num_blocks, num_kv_heads, head_dim, block_size]
 *   x = 16 / sizeof(cache element)          (vasr-paged-attn/src/paged_kv_cache.rs:263-294)
 *
 *   slot_mapping  int64  [num_tokens]; slot = block_id * block_size + offset,
 *                 negative = padding, skipped            (paged_kv_cache.rs:7, 74-103)
 *   block_tables  uint32 [num_seqs, block_table_stride]  (paged_kv_cache.rs:954-964)
 *   context_lens  uint32 [num_seqs]                      (paged_kv_cache.rs:985-1017)
 *   cu_seqlens    uint32 [num_seqs + 1]                  (paged_kv_cache.rs:58-72)
 *
 * Conventions of this ABI:
 *   - All pointers to tensors are device pointers; sizes, strides and scalar
 *     parameters are host values. Strides are in elements.
 *   - Every argument check happens on the host before any launch. A failed
 *     check returns a non-zero status and sets a thread-local message read by
 *     vpa_last_error(). Nothing is launched in that case.
 *   - No entry point allocates device memory, synchronises, or reads device
 *     memory from the host, so every launch may be recorded into a HIP graph.
 *     Scratch memory comes from the caller (see
 *     vpa_paged_attention_workspace_size), except for
 *     vpa_paged_attention_noalloc, which uses a static device array of the
 *     library.
 *   - `stream` is a hipStream_t (NULL = the null stream).
 *   - The library is reentrant; its only global state is the thread-local
 *     error message, a per-device cache of the compute-unit count, and the
 *     per-device decode scratch of vpa_paged_attention_noalloc with its
 *     cached address.
 */
#ifndef VPA_H_
#define VPA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------- */
#define VPA_OK 0
#define VPA_ERR_INVALID_ARGUMENT 1 /* shape, stride, null pointer, mismatch   */
#define VPA_ERR_UNSUPPORTED 2      /* dtype / head_dim / block_size / option  */
#define VPA_ERR_WORKSPACE 3        /* caller workspace too small             */
#define VPA_ERR_HIP 4              /* the HIP runtime reported an error       */
#define VPA_ERR_CAPACITY 5         /* KV pool exhausted (block manager)       */
#define VPA_ERR_NOT_FOUND 6        /* unknown request id (block manager)      */

/* ---- element types --------------------------------------------------- */
#define VPA_DTYPE_F32 0
#define VPA_DTYPE_F16 1
#define VPA_DTYPE_BF16 2
/* OCP E4M3FN, cache element only (the reference's uint8 cache,
 * vasr-paged-attn/src/metal/kernels/prefill_paged_attn.metal:698-722,
 * 1610-1612): 1 byte, x = 16, dequantised as (float)byte * scale. */
#define VPA_DTYPE_FP8_E4M3 3

/* Message of the last failed call on this thread ("" if none). */
const char* vpa_last_error(void);

/* Library version string. */
const char* vpa_version(void);

/*
 * Shapes of one layer's key and value cache for a pool of `num_blocks`
 * blocks. Restates PagedKvCache::new_inner (paged_kv_cache.rs:229-314):
 * x = 16 / dtype_bytes, head_dim must be a multiple of x, every size
 * non-zero. Fills key_shape[5] and value_shape[4].
 *
 * The ops below take head_dim 64, 96, 128, 192 or 256 and block_size 8, 16
 * or 32: the append, the gather and the chunked prefill every combination;
 * decode a (block, head) tile of a whole number of KiB, head_dim *
 * block_size / x a multiple of 64 (head_dim 96 needs 16- or 32-token
 * blocks at 16 bits), and over fp8 caches the shapes listed at
 * vpa_paged_attention. Other shapes return VPA_ERR_UNSUPPORTED.
 */
int vpa_cache_layout(int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                     int64_t num_blocks, int32_t cache_dtype, int64_t* key_shape,
                     int64_t* value_shape);

/*
 * reshape_and_cache — write new K/V rows into the paged cache.
 * Replaces mistralrs_paged_attn::reshape_and_cache(key, value, k_scale,
 * v_scale, key_cache, value_cache, slot_mapping) called at
 * vasr-models/src/model/thinker_text.rs:1101-1109 (decode) and :1324-1332
 * (packed prefill).
 *
 * key/value: [num_tokens, num_kv_heads, head_dim], head stride head_dim, token
 * stride key_token_stride / value_token_stride (>= num_kv_heads*head_dim).
 * For token t with s = slot_mapping[t] >= 0: blk = s / block_size,
 * off = s % block_size,
 *   key_cache  [blk, j, d / x, off, d % x] = key  [t, j, d]
 *   value_cache[blk, j, d, off]            = value[t, j, d]
 * Slots < 0 (PAD_SLOT_ID) and slots >= num_blocks*block_size are skipped.
 * With cache_dtype == dtype the copy is bit-exact and k_scale / v_scale may
 * be NULL (ignored). With cache_dtype VPA_DTYPE_FP8_E4M3 (dtype f32, f16 or
 * bf16) k_scale and v_scale are device pointers to one f32 each and every
 * element is stored as E4M3FN(x / scale), rounded to nearest even and
 * saturated to +-448 (NaN stays NaN) — the rule of the fp8 caches of the
 * reference's paged-attention crate. num_tokens == 0 is a no-op; one call
 * takes at most ceil(num_tokens / block_size) * num_kv_heads < 2^24
 * (VPA_ERR_INVALID_ARGUMENT beyond: split the call).
 *
 * Cache strides: cache_block_stride / cache_head_stride are the element
 * strides of the first two dims of both caches (a (block, head) tile is
 * head_dim*block_size contiguous elements in both).
 */
int vpa_reshape_and_cache(const void* key, const void* value, int64_t key_token_stride,
                          int64_t value_token_stride, const float* k_scale,
                          const float* v_scale, void* key_cache, void* value_cache,
                          const int64_t* slot_mapping, int64_t num_tokens,
                          int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                          int64_t num_blocks, int64_t cache_block_stride,
                          int64_t cache_head_stride, int32_t dtype, int32_t cache_dtype,
                          void* stream);

/*
 * Bytes of caller workspace vpa_paged_attention needs for split-K partials
 * (partial outputs, maxima and sums) at this shape. Depends only on the
 * arguments; 0 is never returned for valid sizes.
 */
size_t vpa_paged_attention_workspace_size(int32_t num_seqs, int32_t num_heads,
                                          int32_t head_dim, int32_t max_context_len);

/*
 * paged_attention — single-token decode over the paged cache.
 * Replaces mistralrs_paged_attn::paged_attention(q, k_scale, v_scale,
 * key_cache, value_cache, block_tables, context_lens, alibi_slopes,
 * max_context_len, softmax_scale, softcapping, sinks) called at
 * vasr-models/src/model/thinker_text.rs:1126-1139.
 *
 * query/out: [num_seqs, num_heads, head_dim] packed, same dtype. For sequence
 * s, q head h, kv head j = h / (num_heads / num_kv_heads)
 * (attention.rs:12-21) and L = min(context_lens[s], max_context_len):
 *   p = softmax_t(softmax_scale * q[s,h] . K[s,j,t]),  t < L
 *   out[s,h] = sum_t p_t V[s,j,t] / (sum_t p_t + 1e-6)  (unnormalised p)
 * where token t lives in block block_tables[s, t / block_size]. Entries
 * >= num_blocks are treated as absent (their tokens are skipped). L == 0
 * gives zeros. max_context_len bounds the split-K grid only (a value frozen
 * at graph capture is fine as long as it is >= every context_len).
 * alibi_slopes and sinks must be NULL and softcapping must be 1.0 (the only
 * values vASR passes); anything else returns VPA_ERR_UNSUPPORTED.
 * Any number of query heads per kv head: the kernels serve 1, 2 or 4 per
 * kv head, and a larger G runs as G / 4 (or / 2, / 1 where 4 does not
 * divide G) replicas of each kv head, each reading that head's tiles.
 * cache_dtype equals dtype, or is VPA_DTYPE_FP8_E4M3 under any query type:
 * K and V are then read as (float)byte * (*k_scale) and
 * (float)byte * (*v_scale), k_scale / v_scale being device pointers to one
 * f32 each (ignored for 16/32-bit caches). Every head_dim of {64, 96, 128,
 * 192, 256} and block_size of {8, 16, 32} is served: the decode kernels
 * take the (block, head) tiles that are whole 1 KiB wave loads (fp8 under
 * 16-bit queries: head_dim 64 or 128 with block_size 16 or 32, 128 or 256
 * with 8, 96 with 32, 192 or 256 with 16 or 32; under f32 queries block_size
 * 16 or 32 with tiles of at most 6 KiB), and the other pairs (16-bit
 * head_dim 96 at block_size 8, the remaining fp8 ones) run on the
 * chunked-prefill vector kernel with one query per sequence, at vector-ALU
 * speed and with the same results contract.
 * workspace must hold vpa_paged_attention_workspace_size(...) bytes (always
 * non-zero for num_seqs > 0: it carries the per-call work list) and be
 * 256-byte aligned. Two calls that run concurrently need two workspaces.
 */
int vpa_paged_attention(void* out, const void* query, const float* k_scale,
                        const float* v_scale, const void* key_cache, const void* value_cache,
                        const uint32_t* block_tables, int32_t block_table_stride,
                        const uint32_t* context_lens, const float* alibi_slopes,
                        int32_t max_context_len, float softmax_scale, float softcapping,
                        const float* sinks, int32_t num_seqs, int32_t num_heads,
                        int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                        int64_t num_blocks, int64_t cache_block_stride,
                        int64_t cache_head_stride, int32_t dtype, int32_t cache_dtype,
                        void* workspace, size_t workspace_bytes, void* stream);

/*
 * paged_attention_plan — build the decode work list of one step into
 * `workspace` once, for the paged_attention calls of every layer of that
 * step (vASR calls paged_attention once per decoder layer with the same
 * block tables and context lengths, thinker_text.rs:1126-1139, so the list
 * is per-step metadata like them). Arguments mean what they mean in
 * vpa_paged_attention (dtype: the query type; the list is the same for
 * every cache type); the workspace is that call's. Stream-ordered and
 * capture-safe; a no-op for configurations whose kernel needs no list.
 * No counterpart in the reference (its decode kernel sizes its grid from
 * max_context_len only).
 */
int vpa_paged_attention_plan(const uint32_t* context_lens, int32_t max_context_len,
                             int32_t block_table_stride, int32_t num_seqs, int32_t num_heads,
                             int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                             int32_t dtype, void* workspace, size_t workspace_bytes,
                             void* stream);

/*
 * paged_attention_planned — vpa_paged_attention without the work-list
 * launch: `workspace` must hold the list that vpa_paged_attention_plan built
 * from the same context_lens contents, max_context_len, block_table_stride,
 * num_seqs and head configuration, earlier in stream order (and no other
 * paged_attention call on that workspace in between). Same arguments,
 * results and errors as vpa_paged_attention. A list that does not match
 * gives wrong results but every memory access stays inside the arguments'
 * bounds.
 */
int vpa_paged_attention_planned(void* out, const void* query, const float* k_scale,
                                const float* v_scale, const void* key_cache,
                                const void* value_cache, const uint32_t* block_tables,
                                int32_t block_table_stride, const uint32_t* context_lens,
                                const float* alibi_slopes, int32_t max_context_len,
                                float softmax_scale, float softcapping, const float* sinks,
                                int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                                int32_t head_dim, int32_t block_size, int64_t num_blocks,
                                int64_t cache_block_stride, int64_t cache_head_stride,
                                int32_t dtype, int32_t cache_dtype, void* workspace,
                                size_t workspace_bytes, void* stream);

/*
 * reshape_and_cache_paged_attention — one decode layer's two calls behind
 * one entry point: reshape_and_cache of the step's new K/V rows
 * (thinker_text.rs:1101-1109) followed by paged_attention
 * (thinker_text.rs:1126-1139), for the decode step where each sequence
 * appends one token at the last position of its context: row s of `key` /
 * `value` ([num_seqs, num_kv_heads, head_dim] of the query type, token
 * strides in elements, heads contiguous) is written at position
 * context_lens[s] - 1 of sequence s's block table, the slot vASR's decode
 * metadata gives that token (paged_kv_cache.rs:985-1017; graph pad rows,
 * context 1 over table row 0, write block 0 offset 0 as slot 0 does). No
 * counterpart in the reference. The results are those of the two calls
 * with that slot mapping, bit for bit (cache bytes and output), provided
 * that no two sequences' last positions share a cache block (vASR's block
 * manager gives each request its own blocks; pad rows share block 0, whose
 * token 0 then holds one of theirs, and each pad row's output is computed
 * over its own token, where the two calls would give all of them the
 * stored one). A sequence with context_lens[s] = 0, or a context that
 * max_context_len or the table clamps, appends nothing.
 * With bf16 / f16 caches (the query's type), a (block, head) tile of 2 to 8
 * KiB (head_dim 64 with blocks of 32 tokens, 128 with 16 or 32, 96 with 32,
 * 192 with 16, 256 with 8 or 16) and at most 48 sequences (the environment variable
 * VPA_FUSED_APPEND_MAX_SEQS, read once, sets another bound), the append runs
 * inside the decode launch: the wave that
 * reads a sequence's last block puts the new token into the K and V tiles
 * it holds and writes whole 32-byte sectors back (the value tile whole, the
 * key units of the token and its sector neighbour). Otherwise (larger
 * batches, where those writes cost the bandwidth-bound decode more than the
 * append's own launch; f32 and fp8 caches; other shapes) it launches the
 * append kernel on the derived slots, then the decode. Arguments and errors
 * as vpa_reshape_and_cache and vpa_paged_attention (dtype: the query and
 * row type; scales as there); softcapping off, no alibi, no sinks.
 */
int vpa_reshape_and_cache_paged_attention(
    void* out, const void* query, const void* key, const void* value, int64_t key_token_stride,
    int64_t value_token_stride, const float* k_scale, const float* v_scale, void* key_cache,
    void* value_cache, const uint32_t* block_tables, int32_t block_table_stride,
    const uint32_t* context_lens, int32_t max_context_len, float softmax_scale, int32_t num_seqs,
    int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
    int64_t num_blocks, int64_t cache_block_stride, int64_t cache_head_stride, int32_t dtype,
    int32_t cache_dtype, void* workspace, size_t workspace_bytes, void* stream);

/*
 * reshape_and_cache_paged_attention_planned — the same without the
 * work-list launch, over the list vpa_paged_attention_plan built (the
 * conditions of vpa_paged_attention_planned).
 */
int vpa_reshape_and_cache_paged_attention_planned(
    void* out, const void* query, const void* key, const void* value, int64_t key_token_stride,
    int64_t value_token_stride, const float* k_scale, const float* v_scale, void* key_cache,
    void* value_cache, const uint32_t* block_tables, int32_t block_table_stride,
    const uint32_t* context_lens, int32_t max_context_len, float softmax_scale, int32_t num_seqs,
    int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
    int64_t num_blocks, int64_t cache_block_stride, int64_t cache_head_stride, int32_t dtype,
    int32_t cache_dtype, void* workspace, size_t workspace_bytes, void* stream);

/*
 * paged_attention_noalloc — vpa_paged_attention with no workspace argument
 * and no allocation of any kind. No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture
 * that must not allocate, tight serving loops, harnesses that forbid
 * hipMalloc). The split-K partials and the work list live in a static
 * device array of the library, 64 MiB per GPU (build-time
 * VPA_NOALLOC_SCRATCH_MIB; `make NOALLOC_SCRATCH_MIB=<n>`), held until the
 * process ends by every process that loads the library, whether or not it
 * calls this entry point, and laid out for the kernel this configuration runs (16-bit / fp8 caches
 * on the rows kernel: num_seqs * num_heads * ceil(max_context_len / 2048)
 * partial rows of (head_dim + 32) floats, 5.3 MB at batch 256 / context
 * 4096, 42 MB at batch 1024 / context 8192). A call whose layout does not
 * fit returns VPA_ERR_WORKSPACE (after the other argument checks, before
 * touching the device). Same arguments (minus the workspace), results and
 * errors as vpa_paged_attention. Every call on a GPU shares that GPU's
 * array. Calls outside stream capture are ordered one after another on each
 * GPU (each call's stream waits for an event recorded after the previous
 * call, on whatever stream): several streams or threads do not race, their
 * calls serialise. Calls captured into a HIP graph are not ordered by the
 * library: the graph's replays must not overlap another use of the array on
 * that GPU. The array's address and the ordering event are set up at the
 * first call on each GPU; no later call creates or allocates anything.
 */
int vpa_paged_attention_noalloc(void* out, const void* query, const float* k_scale,
                                const float* v_scale, const void* key_cache,
                                const void* value_cache, const uint32_t* block_tables,
                                int32_t block_table_stride, const uint32_t* context_lens,
                                const float* alibi_slopes, int32_t max_context_len,
                                float softmax_scale, float softcapping, const float* sinks,
                                int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                                int32_t head_dim, int32_t block_size, int64_t num_blocks,
                                int64_t cache_block_stride, int64_t cache_head_stride,
                                int32_t dtype, int32_t cache_dtype, void* stream);

/*
 * paged_cache_read — a measurement kernel with no counterpart in the
 * reference: reads every K and V byte of each sequence's context through its
 * block table exactly as the decode does (the work list that
 * vpa_paged_attention_plan left in `workspace` for the same lengths and
 * sizes, the same split of each chunk's blocks over the waves, the same
 * 16-byte loads) and computes nothing but an XOR of the bytes. Its rate is
 * the achievable gather bandwidth of the decode's access pattern on the
 * device, the ceiling against which the decode's own rate is read. *sink
 * (device u32) is written only where a lane's checksum equals `magic`.
 * 16-bit or fp8 caches, head_dim <= 128, (block, head) tiles of 1, 2, 4 or
 * 8 KiB.
 */
int vpa_paged_cache_read(const void* key_cache, const void* value_cache,
                         const uint32_t* block_tables, int32_t block_table_stride,
                         int32_t max_context_len, int32_t num_seqs, int32_t num_heads,
                         int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                         int64_t num_blocks, int64_t cache_block_stride,
                         int64_t cache_head_stride, int32_t cache_dtype, void* workspace,
                         size_t workspace_bytes, uint32_t magic, uint32_t* sink, void* stream);

/*
 * gather_kv_cache — copy each sequence's first kv_len tokens out of the paged
 * cache into packed rows.
 * Replaces mistralrs_paged_attn::gather_kv_cache(key_cache, value_cache,
 * k_scale, v_scale, block_tables, cu_seqlens_kv, out_dtype) called at
 * vasr-models/src/model/thinker_text.rs:190-198 and :1344-1352.
 *
 * out_key/out_value: [total_tokens, num_kv_heads, head_dim] packed in
 * out_dtype; row cu_seqlens_kv[s] + t holds token t of sequence s.
 * total_tokens must equal cu_seqlens_kv[num_seqs] (the host knows it from
 * kv_lens). Block ids >= num_blocks produce zero rows. out_dtype equals
 * cache_dtype (bit-exact copy), or the cache is VPA_DTYPE_FP8_E4M3 and
 * out_dtype f32 / f16 / bf16: each value is (float)byte * scale rounded to
 * nearest even, with k_scale / v_scale device pointers to one f32 each.
 * num_seqs and block_table_stride are at most 65535 (VPA_ERR_UNSUPPORTED).
 * Each sequence's kv_len (cu_seqlens_kv[s+1] - cu_seqlens_kv[s]) must not
 * exceed block_table_stride * block_size: the lengths live on the device, so
 * this cannot be checked before the launch, and rows past the table width
 * are left unwritten.
 */
int vpa_gather_kv_cache(void* out_key, void* out_value, const void* key_cache,
                        const void* value_cache, const float* k_scale, const float* v_scale,
                        const uint32_t* block_tables, int32_t block_table_stride,
                        const uint32_t* cu_seqlens_kv, int32_t num_seqs, int64_t total_tokens,
                        int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                        int64_t num_blocks, int64_t cache_block_stride,
                        int64_t cache_head_stride, int32_t cache_dtype, int32_t out_dtype,
                        void* stream);

/*
 * chunked_prefill_paged_attention — causal (or full) varlen attention of the
 * packed prefill queries over the paged cache, without a gathered copy.
 * Replaces the pair gather_kv_cache + attention::run_attention(q, k, v,
 * AttentionMask::None, prefill_flash_params(), scaling, true, groups) of
 * vasr-models/src/model/thinker_text.rs:1344-1365, which runs
 * flash_attn_varlen over the gathered K/V (attention.rs:554-664); with
 * causal = 0 it is also the Metal paged_attention_varlen_prefill(q,
 * key_cache, value_cache, block_tables, context_lens, cu_seqlens_q, k_scale,
 * v_scale, scale, softcapping = 1) of vasr-paged-attn/src/metal/
 * varlen_prefill.rs:284-420.
 *
 * query/out: [total_query_rows, num_heads, head_dim] packed, bf16, f16 or
 * f32 (the reference's flash path takes no f32, attention.rs:562; its Metal
 * prefill does, prefill_paged_attn.metal:1606, 1610). Sequence s owns
 * query rows cu_seqlens_q[s] .. cu_seqlens_q[s+1]-1 (n_s rows) and its first
 * L_s = context_lens[s] cached tokens (PagedInputMetadata::context_lens of a
 * prefill, paged_kv_cache.rs:525-532), the new rows' K/V included (append
 * them with vpa_reshape_and_cache first). With causal
 * != 0, query row i sees keys t <= i + L_s - n_s (bottom-right alignment,
 * attention.rs:78-149); otherwise every t < L_s. A row that sees no key is
 * written as zeros. n_s and L_s are clamped to max_query_len and
 * max_kv_len, which size the grid only; rows at or past total_query_rows are
 * neither read nor written. Block ids >= num_blocks are treated as absent.
 * out[row, h] = sum_t p_t V[t] / (sum_t p_t + denom_eps), p_t = exp(s_t -
 * max_t s_t): denom_eps 0 is the flash attention of the CUDA path, 1e-6 the
 * Metal kernel (prefill_paged_attn.metal:1300); it must be finite and >= 0.
 * Head dims 64, 96, 128, 192 and 256 (the Metal kernel's set,
 * varlen_prefill.rs:15), block_size 8, 16 or 32, any number of query heads
 * per kv head; cache_dtype equals dtype or is VPA_DTYPE_FP8_E4M3 (for any
 * query type). bf16 / f16 queries with 1, 2 or 4 query heads per kv head
 * run on the MFMA kernel where a (block, head) tile is a whole number of
 * 1 KiB DMAs (head_dim 96 at 16- or 32-token blocks for 16 bits, 32-token
 * blocks for fp8; fp8 at 8-token blocks head_dim 128 or 256); every other
 * configuration, f32 included, on a vector-ALU kernel with f32 arithmetic.
 * An fp8 cache is read as byte * k_scale / byte * v_scale (the Metal
 * kernel's fp8 path, prefill_paged_attn.metal:698-769, 797-800), converted
 * to the query type. Needs no workspace; safe under stream capture.
 */
int vpa_chunked_prefill_paged_attention(
    void* out, const void* query, const float* k_scale, const float* v_scale,
    const void* key_cache, const void* value_cache, const uint32_t* block_tables,
    int32_t block_table_stride, const uint32_t* cu_seqlens_q, const uint32_t* context_lens,
    int32_t num_seqs, int32_t max_query_len, int32_t max_kv_len, int64_t total_query_rows,
    float softmax_scale, float denom_eps, int32_t causal, int32_t num_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t block_size, int64_t num_blocks, int64_t cache_block_stride,
    int64_t cache_head_stride, int32_t dtype, int32_t cache_dtype, void* stream);

/*
 * argmax_rows — next-token ids of a batch of logits rows, left on the device.
 * Replaces argmax_token_ids_from_logits(logits, batch)
 * (vasr-models/src/model/generation.rs:443-460: candle argmax over dim 1,
 * then a host read-back of every id), called after each decode forward at
 * vasr-models/src/model/paged_batch_engine.rs:722 and after prefill at :580.
 *
 * logits: [num_rows, row_stride] elements of dtype (f32, f16, bf16), the
 * first `vocab` of each row used. out_ids[r] (u32, device) is the index of
 * the first maximum of row r; NaN values are never chosen, except that a
 * NaN at index 0 gives 0 (candle's left-to-right strictly-greater scan). No
 * host synchronisation; safe under stream capture.
 */
int vpa_argmax_rows(const void* logits, int64_t row_stride, int32_t vocab, int32_t num_rows,
                    int32_t dtype, uint32_t* out_ids, void* stream);

/*
 * decode_consume_tokens — the step-start next-token bookkeeping of the
 * decode loop, on the device. Replaces the host loop of
 * paged_batch_decode_step (vasr-models/src/model/paged_batch_engine.rs:
 * 640-667) that reads the pending ids back: for each row r that is not
 * finished, the pending id next_ids[r] either is an EOS id (one of
 * eos_ids[0..num_eos)) and the row becomes finished, or it is appended to
 * the row's generated list (generated[r, gen_len[r]++], a [num_rows,
 * gen_capacity] u32 buffer; a full list is not extended) and becomes the
 * row's next input id. Finished rows feed eos_fill_id (the reference pads
 * with eos_token_ids[0], paged_batch_engine.rs:193-195) instead of being
 * compacted out of the batch, so a captured decode graph keeps its shape.
 * input_ids[r] receives the row's input id; *active_count the number of rows
 * that fed a real token (the 4 bytes a host loop reads when it checks for
 * completion). finished is u8 per row.
 * prev_slot_mapping (i64 [num_rows], may be NULL) is the previous step's
 * slot_mapping: a row that is not finished and whose previous slot is
 * negative did not run in that step (no block for its token, as
 * try_allocate_slots failing keeps a slot out of the forward,
 * paged_batch_engine.rs:209-227), so it feeds the same input id again,
 * appends nothing and ignores its pending id (the argmax of a forward it
 * took no part in); it counts as active. NULL: every unfinished row
 * consumes its pending id. All pointers are device memory; no host
 * synchronisation; safe under stream capture.
 */
int vpa_decode_consume_tokens(const uint32_t* next_ids, uint8_t* finished,
                              const int64_t* prev_slot_mapping, uint32_t* generated,
                              uint32_t* gen_len, int32_t gen_capacity, const uint32_t* eos_ids,
                              int32_t num_eos, uint32_t eos_fill_id, uint32_t* input_ids,
                              uint32_t* active_count, int32_t num_rows, void* stream);

/*
 * Device-resident KV block allocation (the decode loop without per-step
 * host metadata). State, all device memory, one row per batch slot:
 *   block_tables [num_rows, block_table_stride] u32  each row's blocks, in order
 *   row_blocks   [num_rows] u32   blocks the row holds
 *   positions    [num_rows] u32   position of the row's next token
 *   free_ring    [free_ring_capacity] u32, free_ring_state [2] u32 = {head,
 *                count}: the free block ids in hand-out order (a FIFO ring;
 *                capacity >= the pool's block count)
 * It restates PagedBlockManager (vasr-paged-attn/src/paged_cache_runtime.rs:
 * 217-380: a FIFO free list, initially ids 1..num_blocks-1, handed out from
 * the front, released blocks pushed to the back last block first, block 0
 * never) and decode_metadata_for_batch_step (vasr-paged-attn/src/
 * paged_kv_cache.rs:924-1059). Each call is one launch, safe under stream
 * capture, with no host synchronisation.
 */

/*
 * allocate_rows — grow rows (in index order) to hold target_tokens[r]
 * tokens: a row takes all the blocks it lacks from the ring's head, or none
 * when the ring cannot serve it (ok[r] = 0), as try_allocate_slots row by row
 * (paged_cache_runtime.rs:260-300, paged_batch_engine.rs:209-227). Used to
 * admit requests after prefill.
 */
int vpa_allocate_rows(uint32_t* block_tables, int32_t block_table_stride, uint32_t* row_blocks,
                      const uint32_t* target_tokens, uint8_t* ok, uint32_t* free_ring,
                      uint32_t* free_ring_state, int32_t free_ring_capacity, int32_t block_size,
                      int32_t num_rows, void* stream);

/*
 * decode_step_metadata — one decode step's metadata: for every row not
 * finished (finished may be NULL), in index order, a block is taken from the
 * ring when the row's next token starts one (allocate_slots(prompt_len +
 * step + 1), paged_batch_engine.rs:629-639), then
 *   slot_mapping[r] = block_tables[r, pos / BS] * BS + pos % BS,
 *   context_lens[r] = pos + 1, positions[r] = pos + 1   (pos = positions[r])
 * as decode_metadata_for_batch_step builds them. A row the ring cannot serve,
 * a finished row, or a row whose table is too narrow gets slot_mapping
 * PAD_SLOT_ID (-1) and context_lens 1 and does not advance. status[3] u32 =
 * {rows stalled for lack of blocks, rows rejected (a row may grow by one
 * block per step and must fit block_table_stride), largest context_len}.
 */
int vpa_decode_step_metadata(uint32_t* block_tables, int32_t block_table_stride,
                             uint32_t* row_blocks, uint32_t* positions, const uint8_t* finished,
                             uint32_t* free_ring, uint32_t* free_ring_state,
                             int32_t free_ring_capacity, int32_t block_size,
                             int64_t* slot_mapping, uint32_t* context_lens, uint32_t* status,
                             int32_t num_rows, void* stream);

/*
 * release_blocks — rows (in index order) keep their first keep_blocks[r]
 * blocks and give the rest back to the ring's tail, last block first, id 0
 * never (trim_request_to_num_tokens with keep = ceil(tokens / BS), and
 * free_request with keep = 0; paged_cache_runtime.rs:330-380).
 */
int vpa_release_blocks(const uint32_t* block_tables, int32_t block_table_stride,
                       uint32_t* row_blocks, const uint32_t* keep_blocks, uint32_t* free_ring,
                       uint32_t* free_ring_state, int32_t free_ring_capacity, int32_t num_rows,
                       void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VPA_H_ */
