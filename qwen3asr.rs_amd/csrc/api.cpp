// C-ABI entry points of libvpa: host-side argument checks, then kernel
// launches. Every check runs before anything is launched; a failure returns a
// status code and leaves a message for vpa_last_error().

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <string>

#include "vpa_internal.h"

namespace vpa {

namespace {
thread_local std::string g_last_error;
constexpr int kMaxDevices = 64;
}

int fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error.assign(buf);
  return code;
}

void clear_error() { g_last_error.clear(); }

namespace {

int dtype_bytes(int32_t dtype) {
  switch (dtype) {
    case VPA_DTYPE_F32:
      return 4;
    case VPA_DTYPE_F16:
    case VPA_DTYPE_BF16:
      return 2;
    case VPA_DTYPE_FP8_E4M3:
      return 1;
    default:
      return 0;
  }
}

const char* dtype_name(int32_t dtype) {
  switch (dtype) {
    case VPA_DTYPE_F32:
      return "f32";
    case VPA_DTYPE_F16:
      return "f16";
    case VPA_DTYPE_BF16:
      return "bf16";
    case VPA_DTYPE_FP8_E4M3:
      return "fp8_e4m3";
    default:
      return "unknown";
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool is_float_dtype(int32_t dtype) {
  return dtype == VPA_DTYPE_F32 || dtype == VPA_DTYPE_F16 || dtype == VPA_DTYPE_BF16;
}

// An fp8 cache needs its two scales (device pointers to one f32 each).
int check_scales(const char* op, int32_t cache_dtype, const float* k_scale,
                 const float* v_scale) {
  if (cache_dtype != VPA_DTYPE_FP8_E4M3) return VPA_OK;
  if (k_scale == nullptr || v_scale == nullptr)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: an fp8 cache needs k_scale and v_scale", op);
  if ((reinterpret_cast<uintptr_t>(k_scale) & 3u) != 0 ||
      (reinterpret_cast<uintptr_t>(v_scale) & 3u) != 0)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: k_scale / v_scale must be 4-byte aligned", op);
  return VPA_OK;
}

// Checks shared by every op that reads or writes the paged cache.
int check_cache(const char* op, int32_t cache_dtype, int32_t num_kv_heads, int32_t head_dim,
                int32_t block_size, int64_t num_blocks, int64_t block_stride,
                int64_t head_stride, const void* key_cache, const void* value_cache) {
  const int eb = dtype_bytes(cache_dtype);
  if (eb == 0) return fail(VPA_ERR_UNSUPPORTED, "%s: unsupported cache dtype %d", op, cache_dtype);
  if (num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 || num_blocks <= 0)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: sizes must be positive: num_kv_heads=%d head_dim=%d block_size=%d "
                "num_blocks=%lld",
                op, num_kv_heads, head_dim, block_size, (long long)num_blocks);
  const int x = 16 / eb;
  if (head_dim % x != 0)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: head_dim must be divisible by key cache pack size: head_dim=%d pack=%d", op,
                head_dim, x);
  if (!cache_kernels_supported(cache_dtype, head_dim, block_size))
    return fail(VPA_ERR_UNSUPPORTED,
                "%s: no kernel for dtype=%s head_dim=%d block_size=%d (head_dim in "
                "{64,96,128,192,256}, block_size in {8,16,32})",
                op, dtype_name(cache_dtype), head_dim, block_size);
  const int64_t tile = (int64_t)head_dim * block_size;
  if (head_stride < tile || block_stride < head_stride * num_kv_heads)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: cache strides overlap tiles: block_stride=%lld head_stride=%lld tile=%lld "
                "num_kv_heads=%d",
                op, (long long)block_stride, (long long)head_stride, (long long)tile,
                num_kv_heads);
  if ((head_stride * eb) % 16 != 0 || (block_stride * eb) % 16 != 0)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: cache strides must be multiples of 16 bytes: block_stride=%lld "
                "head_stride=%lld",
                op, (long long)block_stride, (long long)head_stride);
  if (key_cache == nullptr || value_cache == nullptr)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: key_cache and value_cache must be non-null", op);
  if (!aligned16(key_cache) || !aligned16(value_cache))
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: caches must be 16-byte aligned", op);
  return VPA_OK;
}

}  // namespace

int device_cu_count() {
  static std::atomic<int> cache[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) dev = 0;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      n <= 0)
    n = 256;
  cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

namespace {

int hip_status(const char* op, hipError_t e) {
  if (e == hipSuccess) return VPA_OK;
  return fail(VPA_ERR_HIP, "%s: HIP launch failed: %s", op, hipGetErrorString(e));
}

}  // namespace
}  // namespace vpa

using namespace vpa;

extern "C" {

const char* vpa_last_error(void) { return g_last_error.c_str(); }

const char* vpa_version(void) { return "vpa 0.1.0 (gfx950)"; }

int vpa_cache_layout(int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                     int64_t num_blocks, int32_t cache_dtype, int64_t* key_shape,
                     int64_t* value_shape) {
  clear_error();
  if (key_shape == nullptr || value_shape == nullptr)
    return fail(VPA_ERR_INVALID_ARGUMENT, "vpa_cache_layout: shape outputs must be non-null");
  if (num_kv_heads <= 0)
    return fail(VPA_ERR_INVALID_ARGUMENT, "paged kv cache requires at least one kv head");
  if (head_dim <= 0)
    return fail(VPA_ERR_INVALID_ARGUMENT, "paged kv cache requires non-zero head_dim");
  if (block_size <= 0)
    return fail(VPA_ERR_INVALID_ARGUMENT, "paged kv cache requires non-zero block_size");
  if (num_blocks <= 0)
    return fail(VPA_ERR_INVALID_ARGUMENT, "paged kv cache requires non-zero num_blocks");
  const int eb = dtype_bytes(cache_dtype);
  if (eb == 0)
    return fail(VPA_ERR_UNSUPPORTED, "unsupported paged kv cache dtype: %d", cache_dtype);
  const int x = 16 / eb;
  if (head_dim % x != 0)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "head_dim must be divisible by key cache pack size: head_dim=%d pack=%d",
                head_dim, x);
  key_shape[0] = num_blocks;
  key_shape[1] = num_kv_heads;
  key_shape[2] = head_dim / x;
  key_shape[3] = block_size;
  key_shape[4] = x;
  value_shape[0] = num_blocks;
  value_shape[1] = num_kv_heads;
  value_shape[2] = head_dim;
  value_shape[3] = block_size;
  return VPA_OK;
}

int vpa_reshape_and_cache(const void* key, const void* value, int64_t key_token_stride,
                          int64_t value_token_stride, const float* k_scale,
                          const float* v_scale, void* key_cache, void* value_cache,
                          const int64_t* slot_mapping, int64_t num_tokens,
                          int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                          int64_t num_blocks, int64_t cache_block_stride,
                          int64_t cache_head_stride, int32_t dtype, int32_t cache_dtype,
                          void* stream) {
  clear_error();
  const char* op = "reshape_and_cache";
  if (num_tokens < 0) return fail(VPA_ERR_INVALID_ARGUMENT, "%s: num_tokens < 0", op);
  if (!is_float_dtype(dtype))
    return fail(VPA_ERR_UNSUPPORTED, "%s: unsupported input dtype %s", op, dtype_name(dtype));
  if (dtype != cache_dtype && cache_dtype != VPA_DTYPE_FP8_E4M3)
    return fail(VPA_ERR_UNSUPPORTED, "%s: cache dtype %s differs from input dtype %s", op,
                dtype_name(cache_dtype), dtype_name(dtype));
  int rc = check_cache(op, cache_dtype, num_kv_heads, head_dim, block_size, num_blocks,
                       cache_block_stride, cache_head_stride, key_cache, value_cache);
  if (rc != VPA_OK) return rc;
  rc = check_scales(op, cache_dtype, k_scale, v_scale);
  if (rc != VPA_OK) return rc;
  if (num_tokens == 0) return VPA_OK;
  if (key == nullptr || value == nullptr || slot_mapping == nullptr)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: key, value and slot_mapping must be non-null", op);
  const int64_t row = (int64_t)num_kv_heads * head_dim;
  if (key_token_stride < row || value_token_stride < row)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: token stride (key=%lld value=%lld) smaller than num_kv_heads*head_dim=%lld",
                op, (long long)key_token_stride, (long long)value_token_stride, (long long)row);
  const int eb = dtype_bytes(dtype);
  if (!aligned16(key) || !aligned16(value) || (key_token_stride * eb) % 16 != 0 ||
      (value_token_stride * eb) % 16 != 0)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: key/value rows must be 16-byte aligned", op);
  // one 256-lane workgroup per (group of block_size tokens, kv head) on a 1D
  // grid, whose lane count must fit in 32 bits
  if ((num_tokens + block_size - 1) / block_size * num_kv_heads > 0xffffffLL)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: too many tokens for one launch: %lld", op,
                (long long)num_tokens);
  CacheGeom g{num_kv_heads, head_dim, block_size, num_blocks, cache_block_stride,
              cache_head_stride};
  return hip_status(op, launch_reshape_and_cache(dtype, cache_dtype, key, value,
                                                 key_token_stride, value_token_stride,
                                                 key_cache, value_cache, slot_mapping,
                                                 num_tokens, g, k_scale, v_scale,
                                                 static_cast<hipStream_t>(stream)));
}

size_t vpa_paged_attention_workspace_size(int32_t num_seqs, int32_t num_heads,
                                          int32_t head_dim, int32_t max_context_len) {
  return decode_workspace_bytes(num_seqs, num_heads, head_dim, max_context_len);
}

}  // extern "C"

namespace vpa {

// paged_attention and its variants: all checks, then the launch.
int paged_attention_impl(void* out, const void* query, const float* k_scale,
                         const float* v_scale, const void* key_cache,
                         const void* value_cache, const uint32_t* block_tables,
                         int32_t block_table_stride, const uint32_t* context_lens,
                         const float* alibi_slopes, int32_t max_context_len, float softmax_scale,
                         float softcapping, const float* sinks, int32_t num_seqs,
                         int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                         int32_t block_size, int64_t num_blocks, int64_t cache_block_stride,
                         int64_t cache_head_stride, int32_t dtype, int32_t cache_dtype,
                         void* workspace, size_t workspace_bytes, void* stream, bool planned,
                         const DecodeScratch* scratch, const char* op,
                         const DecodeAppend* append) {
  clear_error();
  if (alibi_slopes != nullptr)
    return fail(VPA_ERR_UNSUPPORTED, "%s: alibi_slopes are not supported", op);
  if (sinks != nullptr) return fail(VPA_ERR_UNSUPPORTED, "%s: sinks are not supported", op);
  if (softcapping != 1.0f)
    return fail(VPA_ERR_UNSUPPORTED, "%s: softcapping must be 1.0 (off), got %g", op,
                (double)softcapping);
  const bool fp8 = cache_dtype == VPA_DTYPE_FP8_E4M3;
  if (dtype != cache_dtype &&
      !(fp8 && (dtype == VPA_DTYPE_BF16 || dtype == VPA_DTYPE_F16 || dtype == VPA_DTYPE_F32)))
    return fail(VPA_ERR_UNSUPPORTED, "%s: cache dtype %s differs from query dtype %s", op,
                dtype_name(cache_dtype), dtype_name(dtype));
  int rc = check_cache(op, cache_dtype, num_kv_heads, head_dim, block_size, num_blocks,
                       cache_block_stride, cache_head_stride, key_cache, value_cache);
  if (rc != VPA_OK) return rc;
  rc = check_scales(op, cache_dtype, k_scale, v_scale);
  if (rc != VPA_OK) return rc;
  // The decode kernels take the shapes whose (block, head) tiles are whole
  // 1 KiB wave loads (decode_supported, decode_fp8_shape,
  // decode_f32_fp8_shape); the other head-dim / block-size pairs of the
  // reference's set (16-bit head dim 96 at 8-token blocks; fp8 caches at
  // head dim 64 with 8, 96 with 8 or 16, 192 with 8; under f32 queries
  // 8-token blocks and head dim 256 with 32) run on the chunked-prefill
  // vector kernel, one query per sequence over its whole context, at
  // vector-ALU speed.
  const bool own_kernel =
      fp8 ? (dtype == VPA_DTYPE_F32 ? decode_f32_fp8_shape(head_dim, block_size)
                                    : decode_fp8_shape(head_dim, block_size))
          : decode_supported(dtype, head_dim, block_size, 1);
  const bool on_vector =
      !own_kernel && prefill_vector_supported(dtype, cache_dtype, head_dim, block_size);
  if (!own_kernel && !on_vector)
    return fail(VPA_ERR_UNSUPPORTED,
                "%s: no decode kernel for %s queries over a %s cache at head_dim=%d "
                "block_size=%d (head_dim 64/96/128/192/256, block_size 8/16/32)",
                op, dtype_name(dtype), dtype_name(cache_dtype), head_dim, block_size);
  if (num_seqs < 0 || num_heads <= 0 || max_context_len < 0 || block_table_stride < 0)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: bad sizes num_seqs=%d num_heads=%d max_context_len=%d "
                "block_table_stride=%d",
                op, num_seqs, num_heads, max_context_len, block_table_stride);
  if (num_heads % num_kv_heads != 0)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: num_heads=%d not a multiple of num_kv_heads=%d",
                op, num_heads, num_kv_heads);
  const int group = num_heads / num_kv_heads;
  if (max_context_len > kDecodeMaxPartitions * kDecodeMinPartitionTokens)
    return fail(VPA_ERR_UNSUPPORTED, "%s: max_context_len=%d exceeds %d", op, max_context_len,
                kDecodeMaxPartitions * kDecodeMinPartitionTokens);
  if (num_seqs == 0) return VPA_OK;
  if (num_seqs > 65535)
    return fail(VPA_ERR_UNSUPPORTED, "%s: num_seqs=%d exceeds 65535", op, num_seqs);
  {
    // one workgroup per (sequence, partition, kv head) at most: keep the
    // 1-D grid below 2^25 workgroups
    const int64_t parts =
        std::max<int64_t>(1, ((int64_t)max_context_len + kDecodeMinPartitionTokens - 1) /
                                 kDecodeMinPartitionTokens);
    const int64_t units = (int64_t)num_heads / decode_kernel_group(group);
    if ((int64_t)num_seqs * parts * units > ((int64_t)1 << 25))
      return fail(VPA_ERR_UNSUPPORTED,
                  "%s: num_seqs * ceil(max_context_len/%d) * kv head replicas exceeds 2^25", op,
                  kDecodeMinPartitionTokens);
  }
  if (out == nullptr || query == nullptr || block_tables == nullptr || context_lens == nullptr)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: out, query, block_tables and context_lens must be non-null", op);
  if (!aligned16(out) || !aligned16(query))
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: out and query must be 16-byte aligned", op);
  if (max_context_len > 0 && (int64_t)block_table_stride * block_size < max_context_len)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: block_table_stride=%d too small for max_context_len=%d (block_size=%d)", op,
                block_table_stride, max_context_len, block_size);
  if (append != nullptr) {
    if (append->key == nullptr || append->value == nullptr)
      return fail(VPA_ERR_INVALID_ARGUMENT, "%s: key and value must be non-null", op);
    const int64_t row = (int64_t)num_kv_heads * head_dim;
    if (append->key_token_stride < row || append->value_token_stride < row)
      return fail(VPA_ERR_INVALID_ARGUMENT,
                  "%s: token stride (key=%lld value=%lld) smaller than num_kv_heads*head_dim=%lld",
                  op, (long long)append->key_token_stride, (long long)append->value_token_stride,
                  (long long)row);
    const int eb = dtype_bytes(dtype);
    if (!aligned16(append->key) || !aligned16(append->value) ||
        (append->key_token_stride * eb) % 16 != 0 || (append->value_token_stride * eb) % 16 != 0)
      return fail(VPA_ERR_INVALID_ARGUMENT, "%s: key/value rows must be 16-byte aligned", op);
  }
  const int part_tokens =
      scratch != nullptr ? decode_part_tokens(dtype, head_dim, block_size)
                         : kDecodeMinPartitionTokens;
  const size_t need =
      decode_workspace_bytes(num_seqs, num_heads, head_dim, max_context_len, part_tokens);
  if (scratch != nullptr) {
    if (need > scratch->bytes)
      return fail(VPA_ERR_WORKSPACE,
                  "%s: this call needs %zu bytes of decode scratch, the library's static "
                  "scratch holds %zu (num_seqs=%d num_heads=%d head_dim=%d max_context_len=%d); "
                  "use vpa_paged_attention with a caller workspace",
                  op, need, scratch->bytes, num_seqs, num_heads, head_dim, max_context_len);
    workspace = nullptr;
    workspace_bytes = 0;
    if (need > 0) {
      const int rc_s = scratch->address(op, &workspace);
      if (rc_s != VPA_OK) return rc_s;
      workspace_bytes = scratch->bytes;
    }
  }
  if (need > 0) {
    if (workspace == nullptr || workspace_bytes < need)
      return fail(VPA_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, got %zu", op, need,
                  workspace == nullptr ? (size_t)0 : workspace_bytes);
    if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
      return fail(VPA_ERR_INVALID_ARGUMENT, "%s: workspace must be 256-byte aligned", op);
  }
  CacheGeom g{num_kv_heads, head_dim, block_size, num_blocks, cache_block_stride,
              cache_head_stride};
  DecodeWorkspace ws = carve_decode_workspace(workspace, num_seqs, num_heads, head_dim,
                                              max_context_len, part_tokens);
  ws.planned = planned;
  // The append runs inside the decode launch (the rows kernel's fused form,
  // 16-bit caches) for small batches only: measured on c3's length rule over
  // 28 layers (us per step, two launches against one), batch 1: 226 / 152,
  // 8: 651 / 571, 32: 953 / 889, 64: 1425-1459 / 1459, 128: 2437 / 2524,
  // 256: 4484 / 4721. Inside a bandwidth-bound decode the token's sector
  // writes interleave with the tile reads and cost more than the append's
  // own launch; with few sequences that launch is what costs. Larger batches
  // and the other configurations run the append kernel on the derived slots,
  // then the decode: the same bytes and results either way.
  const bool fuse = append != nullptr &&
                    decode_fuses_append(dtype, cache_dtype, head_dim, block_size, num_seqs, group);
  // the library's scratch orders the calls that share it
  if (scratch != nullptr) {
    const int rc_b = scratch->before(op, stream);
    if (rc_b != VPA_OK) return rc_b;
  }
  int rc_l = VPA_OK;
  if (append != nullptr && !fuse) {
    LastSlots last;
    last.block_tables = block_tables;
    last.context_lens = context_lens;
    last.stride = block_table_stride;
    last.cap = (int32_t)std::min<int64_t>(max_context_len,
                                          (int64_t)block_table_stride * block_size);
    const hipError_t e = launch_append_last_positions(
        dtype, cache_dtype, append->key, append->value, append->key_token_stride,
        append->value_token_stride, const_cast<void*>(key_cache), const_cast<void*>(value_cache),
        last, num_seqs, g, k_scale, v_scale, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) rc_l = hip_status(op, e);
  }
  if (rc_l == VPA_OK && on_vector)
    // one causal query per sequence (row s), the decode's 1e-6 in the
    // denominator
    rc_l = hip_status(op, launch_prefill_vector(
                              dtype, cache_dtype, out, query, key_cache, value_cache,
                              block_tables, block_table_stride, nullptr, context_lens, num_seqs,
                              1, max_context_len, num_seqs, softmax_scale, 1e-6f, 1, num_heads,
                              g, fp8 ? k_scale : nullptr, fp8 ? v_scale : nullptr,
                              static_cast<hipStream_t>(stream)));
  else if (rc_l == VPA_OK)
    rc_l = hip_status(op, launch_paged_decode(dtype, cache_dtype, out, query, key_cache,
                                            value_cache, block_tables, block_table_stride,
                                            context_lens, max_context_len, softmax_scale,
                                            k_scale, v_scale, num_seqs, num_heads, g, ws,
                                            static_cast<hipStream_t>(stream),
                                            fuse ? append : nullptr));
  return scratch != nullptr ? scratch->after(op, stream, rc_l) : rc_l;
}

}  // namespace vpa

extern "C" {

int vpa_paged_attention(void* out, const void* query, const float* k_scale,
                        const float* v_scale, const void* key_cache, const void* value_cache,
                        const uint32_t* block_tables, int32_t block_table_stride,
                        const uint32_t* context_lens, const float* alibi_slopes,
                        int32_t max_context_len, float softmax_scale, float softcapping,
                        const float* sinks, int32_t num_seqs, int32_t num_heads,
                        int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                        int64_t num_blocks, int64_t cache_block_stride,
                        int64_t cache_head_stride, int32_t dtype, int32_t cache_dtype,
                        void* workspace, size_t workspace_bytes, void* stream) {
  return paged_attention_impl(out, query, k_scale, v_scale, key_cache, value_cache,
                              block_tables, block_table_stride, context_lens, alibi_slopes, max_context_len,
                              softmax_scale, softcapping, sinks, num_seqs, num_heads,
                              num_kv_heads, head_dim, block_size, num_blocks, cache_block_stride,
                              cache_head_stride, dtype, cache_dtype, workspace, workspace_bytes,
                              stream, false, nullptr, "paged_attention");
}

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
                                size_t workspace_bytes, void* stream) {
  return paged_attention_impl(out, query, k_scale, v_scale, key_cache, value_cache,
                              block_tables, block_table_stride, context_lens, alibi_slopes, max_context_len,
                              softmax_scale, softcapping, sinks, num_seqs, num_heads,
                              num_kv_heads, head_dim, block_size, num_blocks, cache_block_stride,
                              cache_head_stride, dtype, cache_dtype, workspace, workspace_bytes,
                              stream, true, nullptr, "paged_attention_planned");
}

int vpa_reshape_and_cache_paged_attention(
    void* out, const void* query, const void* key, const void* value, int64_t key_token_stride,
    int64_t value_token_stride, const float* k_scale, const float* v_scale, void* key_cache,
    void* value_cache, const uint32_t* block_tables, int32_t block_table_stride,
    const uint32_t* context_lens, int32_t max_context_len, float softmax_scale, int32_t num_seqs,
    int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
    int64_t num_blocks, int64_t cache_block_stride, int64_t cache_head_stride, int32_t dtype,
    int32_t cache_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  const DecodeAppend app{key, value, key_token_stride, value_token_stride};
  return paged_attention_impl(out, query, k_scale, v_scale, key_cache, value_cache, block_tables,
                              block_table_stride, context_lens, nullptr, max_context_len,
                              softmax_scale, 1.0f, nullptr, num_seqs, num_heads, num_kv_heads,
                              head_dim, block_size, num_blocks, cache_block_stride,
                              cache_head_stride, dtype, cache_dtype, workspace, workspace_bytes,
                              stream, false, nullptr, "reshape_and_cache_paged_attention", &app);
}

int vpa_reshape_and_cache_paged_attention_planned(
    void* out, const void* query, const void* key, const void* value, int64_t key_token_stride,
    int64_t value_token_stride, const float* k_scale, const float* v_scale, void* key_cache,
    void* value_cache, const uint32_t* block_tables, int32_t block_table_stride,
    const uint32_t* context_lens, int32_t max_context_len, float softmax_scale, int32_t num_seqs,
    int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
    int64_t num_blocks, int64_t cache_block_stride, int64_t cache_head_stride, int32_t dtype,
    int32_t cache_dtype, void* workspace, size_t workspace_bytes, void* stream) {
  const DecodeAppend app{key, value, key_token_stride, value_token_stride};
  return paged_attention_impl(out, query, k_scale, v_scale, key_cache, value_cache, block_tables,
                              block_table_stride, context_lens, nullptr, max_context_len,
                              softmax_scale, 1.0f, nullptr, num_seqs, num_heads, num_kv_heads,
                              head_dim, block_size, num_blocks, cache_block_stride,
                              cache_head_stride, dtype, cache_dtype, workspace, workspace_bytes,
                              stream, true, nullptr, "reshape_and_cache_paged_attention_planned",
                              &app);
}

int vpa_paged_attention_plan(const uint32_t* context_lens, int32_t max_context_len,
                             int32_t block_table_stride, int32_t num_seqs, int32_t num_heads,
                             int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                             int32_t dtype, void* workspace, size_t workspace_bytes,
                             void* stream) {
  clear_error();
  const char* op = "paged_attention_plan";
  if (num_seqs < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
      max_context_len < 0 || block_table_stride < 0 || num_heads % num_kv_heads != 0)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: bad sizes num_seqs=%d num_heads=%d num_kv_heads=%d head_dim=%d "
                "block_size=%d max_context_len=%d block_table_stride=%d",
                op, num_seqs, num_heads, num_kv_heads, head_dim, block_size, max_context_len,
                block_table_stride);
  // (shapes the decode kernels do not take run on the chunked-prefill
  // vector kernel, which needs no plan)
  if (!decode_supported(dtype, head_dim, block_size, num_heads / num_kv_heads) &&
      !prefill_vector_supported(dtype, dtype, head_dim, block_size))
    return fail(VPA_ERR_UNSUPPORTED, "%s: no decode kernel for this configuration", op);
  if (max_context_len > kDecodeMaxPartitions * kDecodeMinPartitionTokens)
    return fail(VPA_ERR_UNSUPPORTED, "%s: max_context_len=%d exceeds %d", op, max_context_len,
                kDecodeMaxPartitions * kDecodeMinPartitionTokens);
  if (num_seqs == 0) return VPA_OK;
  if (num_seqs > 65535)
    return fail(VPA_ERR_UNSUPPORTED, "%s: num_seqs=%d exceeds 65535", op, num_seqs);
  if (context_lens == nullptr)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: context_lens must be non-null", op);
  if (max_context_len > 0 && (int64_t)block_table_stride * block_size < max_context_len)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: block_table_stride=%d too small for max_context_len=%d (block_size=%d)", op,
                block_table_stride, max_context_len, block_size);
  const size_t need = decode_workspace_bytes(num_seqs, num_heads, head_dim, max_context_len);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(VPA_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, got %zu", op, need,
                workspace == nullptr ? (size_t)0 : workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: workspace must be 256-byte aligned", op);
  CacheGeom g{num_kv_heads, head_dim, block_size, 1, 0, 0};
  DecodeWorkspace ws =
      carve_decode_workspace(workspace, num_seqs, num_heads, head_dim, max_context_len);
  return hip_status(op, launch_decode_plan(dtype, context_lens, max_context_len,
                                           block_table_stride, num_seqs, g, ws,
                                           static_cast<hipStream_t>(stream)));
}

int vpa_paged_cache_read(const void* key_cache, const void* value_cache,
                         const uint32_t* block_tables, int32_t block_table_stride,
                         int32_t max_context_len, int32_t num_seqs, int32_t num_heads,
                         int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                         int64_t num_blocks, int64_t cache_block_stride,
                         int64_t cache_head_stride, int32_t cache_dtype, void* workspace,
                         size_t workspace_bytes, uint32_t magic, uint32_t* sink, void* stream) {
  clear_error();
  const char* op = "paged_cache_read";
  int rc = check_cache(op, cache_dtype, num_kv_heads, head_dim, block_size, num_blocks,
                       cache_block_stride, cache_head_stride, key_cache, value_cache);
  if (rc != VPA_OK) return rc;
  if (!paged_read_supported(cache_dtype, head_dim, block_size))
    return fail(VPA_ERR_UNSUPPORTED,
                "%s: 16-bit or fp8 caches with head_dim <= 128 and whole-KiB tiles only", op);
  if (num_seqs < 0 || num_heads <= 0 || max_context_len < 0 || block_table_stride < 0)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: bad sizes", op);
  if (num_seqs == 0) return VPA_OK;
  if (num_seqs > 65535)
    return fail(VPA_ERR_UNSUPPORTED, "%s: num_seqs=%d exceeds 65535", op, num_seqs);
  if (max_context_len > kDecodeMaxPartitions * kDecodeMinPartitionTokens)
    return fail(VPA_ERR_UNSUPPORTED, "%s: max_context_len=%d exceeds %d", op, max_context_len,
                kDecodeMaxPartitions * kDecodeMinPartitionTokens);
  if (block_tables == nullptr || sink == nullptr)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: block_tables and sink must be non-null", op);
  if (max_context_len > 0 && (int64_t)block_table_stride * block_size < max_context_len)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: block_table_stride=%d too small for max_context_len=%d (block_size=%d)", op,
                block_table_stride, max_context_len, block_size);
  // the work list that vpa_paged_attention_plan left in the workspace
  const size_t need = decode_workspace_bytes(num_seqs, num_heads, head_dim, max_context_len);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(VPA_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, got %zu", op, need,
                workspace == nullptr ? (size_t)0 : workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: workspace must be 256-byte aligned", op);
  CacheGeom g{num_kv_heads, head_dim, block_size, num_blocks, cache_block_stride,
              cache_head_stride};
  const DecodeWorkspace ws =
      carve_decode_workspace(workspace, num_seqs, num_heads, head_dim, max_context_len);
  return hip_status(op, launch_paged_read(cache_dtype, key_cache, value_cache, block_tables,
                                          block_table_stride, max_context_len, num_seqs, g, ws,
                                          magic, sink, static_cast<hipStream_t>(stream)));
}

int vpa_gather_kv_cache(void* out_key, void* out_value, const void* key_cache,
                        const void* value_cache, const float* k_scale, const float* v_scale,
                        const uint32_t* block_tables, int32_t block_table_stride,
                        const uint32_t* cu_seqlens_kv, int32_t num_seqs, int64_t total_tokens,
                        int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                        int64_t num_blocks, int64_t cache_block_stride,
                        int64_t cache_head_stride, int32_t cache_dtype, int32_t out_dtype,
                        void* stream) {
  clear_error();
  const char* op = "gather_kv_cache";
  if (out_dtype != cache_dtype &&
      !(cache_dtype == VPA_DTYPE_FP8_E4M3 && is_float_dtype(out_dtype)))
    return fail(VPA_ERR_UNSUPPORTED, "%s: out dtype %s differs from cache dtype %s", op,
                dtype_name(out_dtype), dtype_name(cache_dtype));
  int rc = check_cache(op, cache_dtype, num_kv_heads, head_dim, block_size, num_blocks,
                       cache_block_stride, cache_head_stride, key_cache, value_cache);
  if (rc != VPA_OK) return rc;
  rc = check_scales(op, cache_dtype, k_scale, v_scale);
  if (rc != VPA_OK) return rc;
  if (num_seqs < 0 || total_tokens < 0 || block_table_stride < 0)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: bad sizes num_seqs=%d total_tokens=%lld block_table_stride=%d", op, num_seqs,
                (long long)total_tokens, block_table_stride);
  if (num_seqs == 0 || total_tokens == 0 || block_table_stride == 0) return VPA_OK;
  if (num_seqs > 65535 || block_table_stride > 65535)
    return fail(VPA_ERR_UNSUPPORTED,
                "%s: num_seqs=%d and block_table_stride=%d must not exceed 65535", op, num_seqs,
                block_table_stride);
  if (out_key == nullptr || out_value == nullptr || block_tables == nullptr ||
      cu_seqlens_kv == nullptr)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: outputs, block_tables and cu_seqlens_kv must be non-null", op);
  if (!aligned16(out_key) || !aligned16(out_value))
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: outputs must be 16-byte aligned", op);
  CacheGeom g{num_kv_heads, head_dim, block_size, num_blocks, cache_block_stride,
              cache_head_stride};
  return hip_status(op, launch_gather_kv_cache(cache_dtype, out_dtype, out_key, out_value,
                                               key_cache, value_cache, block_tables,
                                               block_table_stride, cu_seqlens_kv, num_seqs, g,
                                               k_scale, v_scale,
                                               static_cast<hipStream_t>(stream)));
}

int vpa_chunked_prefill_paged_attention(
    void* out, const void* query, const float* k_scale, const float* v_scale,
    const void* key_cache, const void* value_cache, const uint32_t* block_tables,
    int32_t block_table_stride, const uint32_t* cu_seqlens_q, const uint32_t* context_lens,
    int32_t num_seqs, int32_t max_query_len, int32_t max_kv_len, int64_t total_query_rows,
    float softmax_scale, float denom_eps, int32_t causal, int32_t num_heads, int32_t num_kv_heads,
    int32_t head_dim, int32_t block_size, int64_t num_blocks, int64_t cache_block_stride,
    int64_t cache_head_stride, int32_t dtype, int32_t cache_dtype, void* stream) {
  clear_error();
  const char* op = "chunked_prefill_paged_attention";
  if (!(denom_eps >= 0.f) || denom_eps > 3.0e38f)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: denom_eps must be finite and >= 0, got %g", op,
                (double)denom_eps);
  const bool fp8 = cache_dtype == VPA_DTYPE_FP8_E4M3;
  if (!is_float_dtype(dtype))
    return fail(VPA_ERR_UNSUPPORTED, "%s: unsupported query dtype %s", op, dtype_name(dtype));
  if (dtype != cache_dtype && !fp8)
    return fail(VPA_ERR_UNSUPPORTED, "%s: cache dtype %s differs from query dtype %s", op,
                dtype_name(cache_dtype), dtype_name(dtype));
  int rc = check_cache(op, cache_dtype, num_kv_heads, head_dim, block_size, num_blocks,
                       cache_block_stride, cache_head_stride, key_cache, value_cache);
  if (rc != VPA_OK) return rc;
  rc = check_scales(op, cache_dtype, k_scale, v_scale);
  if (rc != VPA_OK) return rc;
  if (num_seqs < 0 || num_heads <= 0 || max_query_len < 0 || max_kv_len < 0 ||
      total_query_rows < 0 || block_table_stride < 0)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: bad sizes num_seqs=%d num_heads=%d max_query_len=%d max_kv_len=%d "
                "total_query_rows=%lld block_table_stride=%d",
                op, num_seqs, num_heads, max_query_len, max_kv_len,
                (long long)total_query_rows, block_table_stride);
  if (num_heads % num_kv_heads != 0)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: num_heads=%d not a multiple of num_kv_heads=%d",
                op, num_heads, num_kv_heads);
  const int group = num_heads / num_kv_heads;
  // the MFMA kernel where it is built for the shape, else the vector kernel
  const bool mfma = prefill_supported(dtype, cache_dtype, head_dim, block_size, group);
  if (!mfma && !prefill_vector_supported(dtype, cache_dtype, head_dim, block_size))
    return fail(VPA_ERR_UNSUPPORTED,
                "%s: no kernel for dtype=%s cache=%s head_dim=%d block_size=%d (head_dim "
                "64/96/128/192/256, block_size 8/16/32)",
                op, dtype_name(dtype), dtype_name(cache_dtype), head_dim, block_size);
  if (num_seqs == 0 || max_query_len == 0 || total_query_rows == 0) return VPA_OK;
  {
    const int ppb = prefill_positions_per_workgroup(group);
    const int64_t grid =
        mfma ? (int64_t)num_seqs * ((max_query_len + ppb - 1) / ppb) * (int64_t)num_kv_heads
             : prefill_vector_workgroups(num_seqs, max_query_len, group, num_kv_heads);
    if (grid > ((int64_t)1 << 31) - 1)
      return fail(VPA_ERR_UNSUPPORTED, "%s: grid of %lld workgroups exceeds 2^31-1", op,
                  (long long)grid);
  }
  if (out == nullptr || query == nullptr || block_tables == nullptr ||
      cu_seqlens_q == nullptr || context_lens == nullptr)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: out, query, block_tables, cu_seqlens_q and context_lens must be non-null",
                op);
  if (!aligned16(out) || !aligned16(query))
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: out and query must be 16-byte aligned", op);
  if (max_kv_len > 0 && (int64_t)block_table_stride * block_size < max_kv_len)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: block_table_stride=%d too small for max_kv_len=%d (block_size=%d)", op,
                block_table_stride, max_kv_len, block_size);
  CacheGeom g{num_kv_heads, head_dim, block_size, num_blocks, cache_block_stride,
              cache_head_stride};
  const auto launch = mfma ? launch_prefill_paged : launch_prefill_vector;
  return hip_status(op, launch(dtype, cache_dtype, out, query, key_cache, value_cache,
                               block_tables, block_table_stride, cu_seqlens_q, context_lens,
                               num_seqs, max_query_len, max_kv_len, total_query_rows,
                               softmax_scale, denom_eps, causal, num_heads, g,
                               fp8 ? k_scale : nullptr, fp8 ? v_scale : nullptr,
                               static_cast<hipStream_t>(stream)));
}

int vpa_argmax_rows(const void* logits, int64_t row_stride, int32_t vocab, int32_t num_rows,
                    int32_t dtype, uint32_t* out_ids, void* stream) {
  clear_error();
  const char* op = "argmax_rows";
  if (!is_float_dtype(dtype))
    return fail(VPA_ERR_UNSUPPORTED, "%s: unsupported logits dtype %s", op, dtype_name(dtype));
  if (num_rows < 0 || vocab < 0 || row_stride < vocab)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: bad sizes num_rows=%d vocab=%d row_stride=%lld",
                op, num_rows, vocab, (long long)row_stride);
  if (num_rows == 0) return VPA_OK;
  if (vocab == 0)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: argmax of an empty row (vocab = 0)", op);
  if (logits == nullptr || out_ids == nullptr)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: logits and out_ids must be non-null", op);
  const int eb = dtype_bytes(dtype);
  if ((reinterpret_cast<uintptr_t>(logits) % eb) != 0 ||
      (reinterpret_cast<uintptr_t>(out_ids) & 3u) != 0)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: misaligned pointers", op);
  return hip_status(op, launch_argmax_rows(dtype, logits, row_stride, vocab, num_rows, out_ids,
                                           static_cast<hipStream_t>(stream)));
}

int vpa_decode_consume_tokens(const uint32_t* next_ids, uint8_t* finished,
                              const int64_t* prev_slot_mapping, uint32_t* generated,
                              uint32_t* gen_len, int32_t gen_capacity, const uint32_t* eos_ids,
                              int32_t num_eos, uint32_t eos_fill_id, uint32_t* input_ids,
                              uint32_t* active_count, int32_t num_rows, void* stream) {
  clear_error();
  const char* op = "decode_consume_tokens";
  if (num_rows < 0 || gen_capacity < 0 || num_eos < 0)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: bad sizes num_rows=%d gen_capacity=%d num_eos=%d", op, num_rows,
                gen_capacity, num_eos);
  if (num_eos == 0 || eos_ids == nullptr)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: eos_token_ids is empty", op);
  if (active_count == nullptr)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: active_count must be non-null", op);
  if (num_rows > 0 && (next_ids == nullptr || finished == nullptr || gen_len == nullptr ||
                       input_ids == nullptr || (gen_capacity > 0 && generated == nullptr)))
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: state buffers must be non-null", op);
  return hip_status(op, launch_consume_tokens(next_ids, finished, prev_slot_mapping, generated,
                                              gen_len, gen_capacity, eos_ids, num_eos, eos_fill_id,
                                              input_ids, active_count, num_rows,
                                              static_cast<hipStream_t>(stream)));
}

namespace {
int check_alloc_state(const char* op, const void* block_tables, int32_t stride,
                      const void* row_blocks, const void* ring, const void* ring_state,
                      int32_t ring_cap, int32_t num_rows) {
  if (num_rows < 0 || stride <= 0 || ring_cap <= 0)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: bad sizes num_rows=%d block_table_stride=%d free_ring_capacity=%d", op,
                num_rows, stride, ring_cap);
  if (ring == nullptr || ring_state == nullptr)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: free_ring and free_ring_state must be non-null",
                op);
  if (num_rows > 0 && (block_tables == nullptr || row_blocks == nullptr))
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: block_tables and row_blocks must be non-null",
                op);
  return VPA_OK;
}
}  // namespace

int vpa_allocate_rows(uint32_t* block_tables, int32_t block_table_stride, uint32_t* row_blocks,
                      const uint32_t* target_tokens, uint8_t* ok, uint32_t* free_ring,
                      uint32_t* free_ring_state, int32_t free_ring_capacity, int32_t block_size,
                      int32_t num_rows, void* stream) {
  clear_error();
  const char* op = "allocate_rows";
  int rc = check_alloc_state(op, block_tables, block_table_stride, row_blocks, free_ring,
                             free_ring_state, free_ring_capacity, num_rows);
  if (rc != VPA_OK) return rc;
  if (block_size <= 0) return fail(VPA_ERR_INVALID_ARGUMENT, "%s: block_size must be > 0", op);
  if (num_rows == 0) return VPA_OK;
  if (target_tokens == nullptr || ok == nullptr)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: target_tokens and ok must be non-null", op);
  return hip_status(op, launch_allocate_rows(block_tables, block_table_stride, row_blocks,
                                             target_tokens, ok, free_ring, free_ring_state,
                                             free_ring_capacity, block_size, num_rows,
                                             static_cast<hipStream_t>(stream)));
}

int vpa_decode_step_metadata(uint32_t* block_tables, int32_t block_table_stride,
                             uint32_t* row_blocks, uint32_t* positions, const uint8_t* finished,
                             uint32_t* free_ring, uint32_t* free_ring_state,
                             int32_t free_ring_capacity, int32_t block_size,
                             int64_t* slot_mapping, uint32_t* context_lens, uint32_t* status,
                             int32_t num_rows, void* stream) {
  clear_error();
  const char* op = "decode_step_metadata";
  int rc = check_alloc_state(op, block_tables, block_table_stride, row_blocks, free_ring,
                             free_ring_state, free_ring_capacity, num_rows);
  if (rc != VPA_OK) return rc;
  if (block_size <= 0) return fail(VPA_ERR_INVALID_ARGUMENT, "%s: block_size must be > 0", op);
  if (status == nullptr) return fail(VPA_ERR_INVALID_ARGUMENT, "%s: status must be non-null", op);
  if (num_rows > 0 && (positions == nullptr || slot_mapping == nullptr || context_lens == nullptr))
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: positions, slot_mapping and context_lens must be non-null", op);
  return hip_status(op, launch_decode_step_metadata(
                            block_tables, block_table_stride, row_blocks, positions, finished,
                            free_ring, free_ring_state, free_ring_capacity, block_size,
                            slot_mapping, context_lens, status, num_rows,
                            static_cast<hipStream_t>(stream)));
}

int vpa_release_blocks(const uint32_t* block_tables, int32_t block_table_stride,
                       uint32_t* row_blocks, const uint32_t* keep_blocks, uint32_t* free_ring,
                       uint32_t* free_ring_state, int32_t free_ring_capacity, int32_t num_rows,
                       void* stream) {
  clear_error();
  const char* op = "release_blocks";
  int rc = check_alloc_state(op, block_tables, block_table_stride, row_blocks, free_ring,
                             free_ring_state, free_ring_capacity, num_rows);
  if (rc != VPA_OK) return rc;
  if (num_rows == 0) return VPA_OK;
  if (keep_blocks == nullptr)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: keep_blocks must be non-null", op);
  return hip_status(op, launch_release_blocks(block_tables, block_table_stride, row_blocks,
                                              keep_blocks, free_ring, free_ring_state,
                                              free_ring_capacity, num_rows,
                                              static_cast<hipStream_t>(stream)));
}

}  // extern "C"
