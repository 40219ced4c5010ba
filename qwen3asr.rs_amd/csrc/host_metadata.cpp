// Host-side bookkeeping of the paged KV cache (include/vpa_host.h): pool
// sizing, the block manager, the per-step metadata builders and the
// decode-graph padding rules of vasr-paged-attn
// (src/paged_cache_runtime.rs, src/paged_kv_cache.rs, src/cuda_graph.rs),
// written as plain C++ over caller-owned arrays.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <deque>
#include <limits>
#include <new>
#include <unordered_map>
#include <vector>

#include "../../include/vpa_host.h"
#include "vpa_internal.h"
#include "vpa_internal.h"

struct vpa_block_manager {
  int32_t block_size = 0;
  std::deque<uint32_t> free_list;                               // front = next to hand out
  std::unordered_map<uint64_t, std::vector<uint32_t>> requests;  // request -> its blocks
};

namespace vpa {
namespace {

constexpr int64_t kPadSlotId = -1;        // PAD_SLOT_ID, paged_kv_cache.rs:7
constexpr int64_t kGraphContextBucketTokens = 256;  // cuda_graph.rs:17
constexpr int32_t kGraphMaxBatch = 256;             // cuda_graph.rs:19

int64_t div_ceil(int64_t a, int64_t b) { return (a + b - 1) / b; }

int elem_size(int32_t dtype) {
  switch (dtype) {
    case VPA_DTYPE_F32:
      return 4;
    case VPA_DTYPE_F16:
    case VPA_DTYPE_BF16:
      return 2;
    default:
      return 0;
  }
}

// Shared argument checks of the ragged block-table builders.
int check_tables(const char* op, const uint32_t* tables, int32_t stride, const int32_t* table_lens,
                 int32_t batch, int32_t block_size, int64_t num_blocks, int32_t* max_len) {
  if (batch <= 0) return fail(VPA_ERR_INVALID_ARGUMENT, "%s: paged metadata batch must be non-empty", op);
  if (block_size <= 0 || num_blocks <= 0)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: block_size and num_blocks must be positive", op);
  if (table_lens == nullptr || (tables == nullptr && stride > 0))
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: block tables must be non-null", op);
  int32_t m = 0;
  for (int32_t s = 0; s < batch; ++s) {
    if (table_lens[s] < 0 || table_lens[s] > stride)
      return fail(VPA_ERR_INVALID_ARGUMENT, "%s: table_lens[%d]=%d outside [0, stride=%d]", op, s,
                  table_lens[s], stride);
    m = std::max(m, table_lens[s]);
  }
  if (m == 0)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: paged metadata requires at least one block per sequence", op);
  *max_len = m;
  return VPA_OK;
}

int slot_of(const char* op, const uint32_t* table, int32_t table_len, int32_t seq,
            int32_t block_size, int64_t num_blocks, int64_t position, int64_t* slot) {
  if (position < 0)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: negative position %lld", op, (long long)position);
  const int64_t block_idx = position / block_size;
  const int64_t offset = position % block_size;
  if (block_idx >= table_len)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: missing block table entry: sequence=%d block_idx=%lld position=%lld "
                "block_size=%d table_len=%d",
                op, seq, (long long)block_idx, (long long)position, block_size, table_len);
  const uint32_t block_id = table[block_idx];
  if ((int64_t)block_id >= num_blocks)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: block id exceeds paged cache capacity: block_id=%u num_blocks=%lld", op,
                block_id, (long long)num_blocks);
  *slot = (int64_t)block_id * block_size + offset;
  return VPA_OK;
}

int write_tables(const char* op, const uint32_t* tables, int32_t stride, const int32_t* table_lens,
                 int32_t batch, int32_t max_len, vpa_paged_metadata* out) {
  if (out->block_tables == nullptr) return VPA_OK;
  if (out->cols < max_len)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: out cols=%d below the longest table (%d)", op,
                out->cols, max_len);
  for (int32_t s = 0; s < batch; ++s) {
    uint32_t* row = out->block_tables + (int64_t)s * out->cols;
    for (int32_t c = 0; c < out->cols; ++c)
      row[c] = c < table_lens[s] ? tables[(int64_t)s * stride + c] : 0u;
  }
  return VPA_OK;
}

int to_u32(const char* op, int64_t v, uint32_t* o) {
  if (v < 0 || v > (int64_t)std::numeric_limits<uint32_t>::max())
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: length overflows u32: %lld", op, (long long)v);
  *o = (uint32_t)v;
  return VPA_OK;
}

int cumulative(const char* op, const int64_t* lengths, int32_t n, uint32_t* cu) {
  uint64_t total = 0;
  if (cu != nullptr) cu[0] = 0;
  for (int32_t i = 0; i < n; ++i) {
    if (lengths[i] < 0 || lengths[i] > (int64_t)std::numeric_limits<uint32_t>::max())
      return fail(VPA_ERR_INVALID_ARGUMENT, "%s: sequence length overflows u32: %lld", op,
                  (long long)lengths[i]);
    total += (uint64_t)lengths[i];
    if (total > std::numeric_limits<uint32_t>::max())
      return fail(VPA_ERR_INVALID_ARGUMENT, "%s: cumulative sequence length overflow", op);
    if (cu != nullptr) cu[i + 1] = (uint32_t)total;
  }
  return VPA_OK;
}

// cu_seqlens and maxima of build_varlen_metadata (paged_kv_cache.rs:105-146).
int varlen(const char* op, const std::vector<int64_t>& q, const std::vector<int64_t>& kv,
           vpa_paged_metadata* out) {
  int rc = cumulative(op, q.data(), (int32_t)q.size(), out->cu_seqlens_q);
  if (rc != VPA_OK) return rc;
  rc = cumulative(op, kv.data(), (int32_t)kv.size(), out->cu_seqlens_kv);
  if (rc != VPA_OK) return rc;
  out->max_query_len = q.empty() ? 0 : *std::max_element(q.begin(), q.end());
  out->max_kv_len = kv.empty() ? 0 : *std::max_element(kv.begin(), kv.end());
  return VPA_OK;
}

}  // namespace
}  // namespace vpa

using namespace vpa;

extern "C" {

int vpa_bytes_per_paged_block(int32_t num_layers, int32_t num_kv_heads, int32_t head_dim,
                              int32_t block_size, int32_t dtype, uint64_t* bytes) {
  clear_error();
  const char* op = "bytes_per_paged_block";
  if (num_layers <= 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: paged block sizing requires non-zero layer/head/block parameters", op);
  const int eb = elem_size(dtype);
  if (eb == 0) return fail(VPA_ERR_UNSUPPORTED, "%s: unsupported paged kv cache dtype %d", op, dtype);
  if (bytes == nullptr) return fail(VPA_ERR_INVALID_ARGUMENT, "%s: bytes must be non-null", op);
  *bytes = (uint64_t)num_layers * num_kv_heads * head_dim * block_size * 2u * eb;
  return VPA_OK;
}

int vpa_pool_blocks_for_context(int64_t tokens, int32_t block_size, int64_t* num_blocks) {
  clear_error();
  if (tokens < 0 || block_size <= 0 || num_blocks == nullptr)
    return fail(VPA_ERR_INVALID_ARGUMENT, "pool_blocks_for_context: bad arguments tokens=%lld "
                "block_size=%d", (long long)tokens, block_size);
  *num_blocks = div_ceil(tokens, block_size) + 1;
  return VPA_OK;
}

int vpa_pool_blocks_for_byte_budget(uint64_t byte_budget, uint64_t bytes_per_block,
                                    int64_t* num_blocks) {
  clear_error();
  const char* op = "pool_blocks_for_byte_budget";
  if (num_blocks == nullptr) return fail(VPA_ERR_INVALID_ARGUMENT, "%s: null output", op);
  if (bytes_per_block == 0)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: paged block byte size must be non-zero", op);
  const uint64_t n = byte_budget / bytes_per_block + 1;
  if (n <= 1)
    return fail(VPA_ERR_CAPACITY,
                "%s: paged KV byte budget %llu is too small for one block (%llu bytes)", op,
                (unsigned long long)byte_budget, (unsigned long long)bytes_per_block);
  *num_blocks = (int64_t)n;
  return VPA_OK;
}

int vpa_pool_blocks_for_memory_fraction(float fraction, uint64_t bytes_per_block,
                                        int64_t* num_blocks) {
  clear_error();
  const char* op = "pool_blocks_for_memory_fraction";
  if (!(fraction > 0.f && fraction <= 1.f))
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: GPU memory fraction must be in (0.0, 1.0]; got %g",
                op, (double)fraction);
  // the library's device code (and with it the static decode scratch of the
  // allocation-free entry point) is loaded first, so that the free memory
  // read below already excludes it
  const int rc_load = vpa::load_device_code(op);
  if (rc_load != VPA_OK) return rc_load;
  size_t free_b = 0, total_b = 0;
  const hipError_t e = hipMemGetInfo(&free_b, &total_b);
  if (e != hipSuccess)
    return fail(VPA_ERR_HIP, "%s: hipMemGetInfo failed: %s", op, hipGetErrorString(e));
  const uint64_t total_mib = (uint64_t)total_b >> 20;
  const uint64_t used_mib = (uint64_t)(total_b - free_b) >> 20;
  const uint64_t target_mib = (uint64_t)std::floor((double)total_mib * (double)fraction);
  const uint64_t budget_mib = target_mib > used_mib ? target_mib - used_mib : 0;
  if (budget_mib == 0)
    return fail(VPA_ERR_CAPACITY,
                "%s: GPU KV budget exhausted: total_mib=%llu used_mib=%llu fraction=%g", op,
                (unsigned long long)total_mib, (unsigned long long)used_mib, (double)fraction);
  return vpa_pool_blocks_for_byte_budget(budget_mib << 20, bytes_per_block, num_blocks);
}

int vpa_block_manager_create(int64_t num_blocks, int32_t block_size, vpa_block_manager** out) {
  clear_error();
  const char* op = "block_manager_create";
  if (out == nullptr) return fail(VPA_ERR_INVALID_ARGUMENT, "%s: null output", op);
  *out = nullptr;
  if (num_blocks <= 0 || block_size <= 0 ||
      num_blocks > (int64_t)std::numeric_limits<uint32_t>::max() + 1)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: bad sizes num_blocks=%lld block_size=%d", op,
                (long long)num_blocks, block_size);
  vpa_block_manager* m = new (std::nothrow) vpa_block_manager();
  if (m == nullptr) return fail(VPA_ERR_CAPACITY, "%s: out of host memory", op);
  m->block_size = block_size;
  try {
    for (int64_t id = 1; id < num_blocks; ++id) m->free_list.push_back((uint32_t)id);
  } catch (const std::bad_alloc&) {
    delete m;
    return fail(VPA_ERR_CAPACITY, "%s: out of host memory", op);
  }
  *out = m;
  return VPA_OK;
}

void vpa_block_manager_destroy(vpa_block_manager* manager) { delete manager; }

int64_t vpa_block_manager_free_blocks(const vpa_block_manager* manager) {
  return manager == nullptr ? 0 : (int64_t)manager->free_list.size();
}

int64_t vpa_block_manager_blocks_for_request(const vpa_block_manager* manager,
                                             uint64_t request_id) {
  if (manager == nullptr) return 0;
  auto it = manager->requests.find(request_id);
  return it == manager->requests.end() ? 0 : (int64_t)it->second.size();
}

int64_t vpa_block_manager_total_allocated_blocks(const vpa_block_manager* manager) {
  if (manager == nullptr) return 0;
  int64_t n = 0;
  for (const auto& kv : manager->requests) n += (int64_t)kv.second.size();
  return n;
}

int vpa_block_manager_slots_available(const vpa_block_manager* manager, uint64_t request_id,
                                      int64_t num_tokens) {
  if (manager == nullptr || num_tokens < 0) return 0;
  const int64_t required = div_ceil(num_tokens, manager->block_size);
  const int64_t existing = vpa_block_manager_blocks_for_request(manager, request_id);
  const int64_t needed = std::max<int64_t>(0, required - existing);
  return needed <= (int64_t)manager->free_list.size() ? 1 : 0;
}

int vpa_block_manager_try_allocate(vpa_block_manager* manager, uint64_t request_id,
                                   int64_t num_tokens, int32_t* allocated) {
  clear_error();
  const char* op = "block_manager_try_allocate";
  if (manager == nullptr || allocated == nullptr || num_tokens < 0)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: bad arguments", op);
  const int64_t required = div_ceil(num_tokens, manager->block_size);
  const int64_t existing = vpa_block_manager_blocks_for_request(manager, request_id);
  const int64_t needed = std::max<int64_t>(0, required - existing);
  *allocated = 1;
  if (needed == 0) return VPA_OK;
  if (needed > (int64_t)manager->free_list.size()) {
    *allocated = 0;
    return VPA_OK;
  }
  try {
    std::vector<uint32_t>& blocks = manager->requests[request_id];
    blocks.reserve((size_t)required);
    for (int64_t i = 0; i < needed; ++i) {
      blocks.push_back(manager->free_list.front());
      manager->free_list.pop_front();
    }
  } catch (const std::bad_alloc&) {
    return fail(VPA_ERR_CAPACITY, "%s: out of host memory", op);
  }
  return VPA_OK;
}

int vpa_block_manager_allocate(vpa_block_manager* manager, uint64_t request_id,
                               int64_t num_tokens) {
  int32_t ok = 0;
  const int rc = vpa_block_manager_try_allocate(manager, request_id, num_tokens, &ok);
  if (rc != VPA_OK) return rc;
  if (!ok)
    return fail(VPA_ERR_CAPACITY,
                "paged KV cache exhausted: request_id=%llu num_tokens=%lld free_blocks=%lld",
                (unsigned long long)request_id, (long long)num_tokens,
                (long long)manager->free_list.size());
  return VPA_OK;
}

int vpa_block_manager_trim(vpa_block_manager* manager, uint64_t request_id, int64_t num_tokens) {
  clear_error();
  if (manager == nullptr || num_tokens < 0)
    return fail(VPA_ERR_INVALID_ARGUMENT, "block_manager_trim: bad arguments");
  auto it = manager->requests.find(request_id);
  if (it == manager->requests.end()) return VPA_OK;
  const size_t keep = (size_t)div_ceil(num_tokens, manager->block_size);
  std::vector<uint32_t>& blocks = it->second;
  if (keep >= blocks.size()) return VPA_OK;
  // the tail returns to the back of the free list, last block first
  for (size_t i = blocks.size(); i-- > keep;)
    if (blocks[i] != 0u) manager->free_list.push_back(blocks[i]);
  blocks.resize(keep);
  return VPA_OK;
}

int vpa_block_manager_free_request(vpa_block_manager* manager, uint64_t request_id) {
  clear_error();
  if (manager == nullptr) return fail(VPA_ERR_INVALID_ARGUMENT, "block_manager_free_request: null");
  auto it = manager->requests.find(request_id);
  if (it == manager->requests.end()) return VPA_OK;
  const std::vector<uint32_t>& blocks = it->second;
  for (size_t i = blocks.size(); i-- > 0;)
    if (blocks[i] != 0u) manager->free_list.push_back(blocks[i]);
  manager->requests.erase(it);
  return VPA_OK;
}

int vpa_block_manager_block_ids(const vpa_block_manager* manager, uint64_t request_id,
                                uint32_t* ids, int64_t capacity, int64_t* count) {
  clear_error();
  const char* op = "block_manager_block_ids";
  if (manager == nullptr || count == nullptr)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: bad arguments", op);
  auto it = manager->requests.find(request_id);
  if (it == manager->requests.end()) {
    *count = 0;
    return fail(VPA_ERR_NOT_FOUND, "%s: paged KV request has no allocated blocks: request_id=%llu",
                op, (unsigned long long)request_id);
  }
  const std::vector<uint32_t>& blocks = it->second;
  *count = (int64_t)blocks.size();
  if ((int64_t)blocks.size() > capacity || (ids == nullptr && !blocks.empty()))
    return fail(VPA_ERR_CAPACITY, "%s: %zu ids do not fit capacity %lld", op, blocks.size(),
                (long long)capacity);
  std::copy(blocks.begin(), blocks.end(), ids);
  return VPA_OK;
}

int vpa_block_manager_block_tables(const vpa_block_manager* manager, const uint64_t* request_ids,
                                   int32_t num_requests, int32_t cols, uint32_t* tables,
                                   int32_t* table_lens) {
  clear_error();
  const char* op = "block_manager_block_tables";
  if (manager == nullptr || num_requests < 0 || cols < 0 ||
      (num_requests > 0 && (request_ids == nullptr || tables == nullptr || table_lens == nullptr)))
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: bad arguments", op);
  for (int32_t r = 0; r < num_requests; ++r) {
    auto it = manager->requests.find(request_ids[r]);
    if (it == manager->requests.end())
      return fail(VPA_ERR_NOT_FOUND,
                  "%s: paged KV request has no allocated blocks: request_id=%llu", op,
                  (unsigned long long)request_ids[r]);
    if ((int64_t)it->second.size() > cols)
      return fail(VPA_ERR_CAPACITY, "%s: request %llu has %zu blocks, cols=%d", op,
                  (unsigned long long)request_ids[r], it->second.size(), cols);
  }
  for (int32_t r = 0; r < num_requests; ++r) {
    const std::vector<uint32_t>& blocks = manager->requests.find(request_ids[r])->second;
    uint32_t* row = tables + (int64_t)r * cols;
    for (int32_t c = 0; c < cols; ++c) row[c] = c < (int32_t)blocks.size() ? blocks[c] : 0u;
    table_lens[r] = (int32_t)blocks.size();
  }
  return VPA_OK;
}

int vpa_slot_for_block_table_position(const uint32_t* table, int32_t table_len,
                                      int32_t block_size, int64_t num_blocks, int64_t position,
                                      int64_t* slot) {
  clear_error();
  const char* op = "slot_for_block_table_position";
  if (slot == nullptr || block_size <= 0 || table_len < 0 || (table == nullptr && table_len > 0))
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: bad arguments", op);
  return slot_of(op, table, table_len, 0, block_size, num_blocks, position, slot);
}

int vpa_cumulative_seqlens(const int64_t* lengths, int32_t n, uint32_t* cu) {
  clear_error();
  if (n < 0 || cu == nullptr || (lengths == nullptr && n > 0))
    return fail(VPA_ERR_INVALID_ARGUMENT, "cumulative_seqlens: bad arguments");
  return cumulative("cumulative_seqlens", lengths, n, cu);
}

int vpa_metadata_from_block_tables(const uint32_t* tables, int32_t stride,
                                   const int32_t* table_lens, int32_t batch,
                                   const int64_t* starts, int32_t len,
                                   const int64_t* context_lens, int32_t block_size,
                                   int64_t num_blocks, vpa_paged_metadata* out) {
  clear_error();
  const char* op = "metadata_from_block_tables";
  int32_t max_len = 0;
  int rc = check_tables(op, tables, stride, table_lens, batch, block_size, num_blocks, &max_len);
  if (rc != VPA_OK) return rc;
  if (out == nullptr || starts == nullptr || context_lens == nullptr || len < 0 ||
      (out->slot_mapping == nullptr && len > 0) || out->context_lens == nullptr)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: bad arguments", op);
  for (int32_t s = 0; s < batch; ++s)
    for (int32_t i = 0; i < len; ++i) {
      rc = slot_of(op, tables + (int64_t)s * stride, table_lens[s], s, block_size, num_blocks,
                   starts[s] + i, &out->slot_mapping[(int64_t)s * len + i]);
      if (rc != VPA_OK) return rc;
    }
  rc = write_tables(op, tables, stride, table_lens, batch, max_len, out);
  if (rc != VPA_OK) return rc;
  int64_t max_ctx = 0;
  for (int32_t s = 0; s < batch; ++s) {
    rc = to_u32(op, context_lens[s], &out->context_lens[s]);
    if (rc != VPA_OK) return rc;
    max_ctx = std::max(max_ctx, context_lens[s]);
  }
  out->num_tokens = (int64_t)batch * len;
  out->max_context_len = max_ctx;
  out->causal_only = 0;
  return varlen(op, std::vector<int64_t>(batch, len),
                std::vector<int64_t>(context_lens, context_lens + batch), out);
}

int vpa_metadata_from_attention_masks(const uint32_t* tables, int32_t stride,
                                      const int32_t* table_lens, int32_t batch,
                                      const uint32_t* masks, int32_t seq_len, int32_t block_size,
                                      int64_t num_blocks, vpa_paged_metadata* out) {
  clear_error();
  const char* op = "metadata_from_attention_masks";
  if (batch <= 0) return fail(VPA_ERR_INVALID_ARGUMENT, "%s: paged metadata batch must be non-empty", op);
  if (seq_len <= 0) return fail(VPA_ERR_INVALID_ARGUMENT, "%s: attention mask rows must be non-empty", op);
  int32_t max_len = 0;
  int rc = check_tables(op, tables, stride, table_lens, batch, block_size, num_blocks, &max_len);
  if (rc != VPA_OK) return rc;
  if (out == nullptr || masks == nullptr || out->slot_mapping == nullptr ||
      out->context_lens == nullptr)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: bad arguments", op);
  std::vector<int64_t> lens(batch, 0);
  bool causal_only = true;
  for (int32_t s = 0; s < batch; ++s) {
    for (int32_t p = 0; p < seq_len; ++p) {
      int64_t* slot = &out->slot_mapping[(int64_t)s * seq_len + p];
      if (masks[(int64_t)s * seq_len + p] == 0u) {
        *slot = kPadSlotId;
        continue;
      }
      rc = slot_of(op, tables + (int64_t)s * stride, table_lens[s], s, block_size, num_blocks, p,
                   slot);
      if (rc != VPA_OK) return rc;
      ++lens[s];
    }
    rc = to_u32(op, lens[s], &out->context_lens[s]);
    if (rc != VPA_OK) return rc;
    causal_only = causal_only && lens[s] == seq_len;
  }
  rc = write_tables(op, tables, stride, table_lens, batch, max_len, out);
  if (rc != VPA_OK) return rc;
  out->num_tokens = (int64_t)batch * seq_len;
  out->max_context_len = *std::max_element(lens.begin(), lens.end());
  out->causal_only = causal_only ? 1 : 0;
  return varlen(op, lens, lens, out);
}

int vpa_metadata_from_query_lens(const uint32_t* tables, int32_t stride,
                                 const int32_t* table_lens, int32_t batch,
                                 const int64_t* query_lens, int32_t block_size,
                                 int64_t num_blocks, vpa_paged_metadata* out) {
  clear_error();
  const char* op = "metadata_from_query_lens";
  if (batch <= 0) return fail(VPA_ERR_INVALID_ARGUMENT, "%s: paged metadata batch must be non-empty", op);
  int32_t max_len = 0;
  int rc = check_tables(op, tables, stride, table_lens, batch, block_size, num_blocks, &max_len);
  if (rc != VPA_OK) return rc;
  if (out == nullptr || query_lens == nullptr || out->slot_mapping == nullptr ||
      out->context_lens == nullptr)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: bad arguments", op);
  int64_t total = 0;
  for (int32_t s = 0; s < batch; ++s) {
    if (query_lens[s] <= 0)
      return fail(VPA_ERR_INVALID_ARGUMENT, "%s: packed prefill query length must be non-zero", op);
    total += query_lens[s];
  }
  int64_t t = 0;
  for (int32_t s = 0; s < batch; ++s) {
    for (int64_t p = 0; p < query_lens[s]; ++p) {
      rc = slot_of(op, tables + (int64_t)s * stride, table_lens[s], s, block_size, num_blocks, p,
                   &out->slot_mapping[t++]);
      if (rc != VPA_OK) return rc;
    }
    if (table_lens[s] < div_ceil(query_lens[s], block_size))
      return fail(VPA_ERR_INVALID_ARGUMENT,
                  "%s: paged block table too short for packed prefill: seq=%d len=%lld have=%d",
                  op, s, (long long)query_lens[s], table_lens[s]);
    rc = to_u32(op, query_lens[s], &out->context_lens[s]);
    if (rc != VPA_OK) return rc;
  }
  rc = write_tables(op, tables, stride, table_lens, batch, max_len, out);
  if (rc != VPA_OK) return rc;
  std::vector<int64_t> lens(query_lens, query_lens + batch);
  out->num_tokens = total;
  out->max_context_len = *std::max_element(lens.begin(), lens.end());
  out->causal_only = 1;
  return varlen(op, lens, lens, out);
}

int vpa_decode_metadata_for_batch_steps(const uint32_t* tables, int32_t stride,
                                        const int32_t* table_lens, int32_t batch,
                                        const int64_t* prompt_lens, int32_t steps,
                                        int32_t block_size, int64_t num_blocks,
                                        int64_t max_tokens_per_sequence, int32_t graph_buckets,
                                        int32_t cols, int64_t* slots, uint32_t* context_lens,
                                        int64_t* max_context_lens, uint32_t* block_tables) {
  clear_error();
  const char* op = "decode_metadata_for_batch_steps";
  if (batch <= 0)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: paged batch decode metadata requires at least one sequence", op);
  int32_t max_len = 0;
  int rc = check_tables(op, tables, stride, table_lens, batch, block_size, num_blocks, &max_len);
  if (rc != VPA_OK) return rc;
  if (prompt_lens == nullptr || steps < 0 || (steps > 0 && (slots == nullptr ||
      context_lens == nullptr || max_context_lens == nullptr)))
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: bad arguments", op);
  const int64_t width =
      graph_buckets ? vpa_bucket_block_table_cols(max_len, block_size) : (int64_t)max_len;
  if (block_tables != nullptr) {
    if (cols < width)
      return fail(VPA_ERR_INVALID_ARGUMENT, "%s: cols=%d below the table width %lld", op, cols,
                  (long long)width);
    vpa_paged_metadata m{};
    m.block_tables = block_tables;
    m.cols = cols;
    rc = write_tables(op, tables, stride, table_lens, batch, max_len, &m);
    if (rc != VPA_OK) return rc;
  }
  for (int32_t t = 0; t < steps; ++t) {
    int64_t step_max = 0;
    for (int32_t s = 0; s < batch; ++s) {
      const int64_t position = prompt_lens[s] + t;
      const int64_t ctx = position + 1;
      if (ctx > max_tokens_per_sequence)
        return fail(VPA_ERR_CAPACITY,
                    "%s: batch decode context length exceeds paged kv cache sequence capacity: "
                    "context_len=%lld max_tokens_per_sequence=%lld",
                    op, (long long)ctx, (long long)max_tokens_per_sequence);
      rc = slot_of(op, tables + (int64_t)s * stride, table_lens[s], s, block_size, num_blocks,
                   position, &slots[(int64_t)t * batch + s]);
      if (rc != VPA_OK) return rc;
      rc = to_u32(op, ctx, &context_lens[(int64_t)t * batch + s]);
      if (rc != VPA_OK) return rc;
      step_max = std::max(step_max, ctx);
    }
    max_context_lens[t] = step_max;
  }
  return VPA_OK;
}

int vpa_contiguous_slot(int64_t sequence, int64_t position, int64_t batch,
                        int64_t blocks_per_sequence, int32_t block_size,
                        int64_t max_tokens_per_sequence, int64_t* slot) {
  clear_error();
  const char* op = "contiguous_slot";
  if (slot == nullptr || block_size <= 0 || sequence < 0 || position < 0)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: bad arguments", op);
  if (sequence >= batch)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: sequence exceeds paged kv cache batch: sequence=%lld batch=%lld", op,
                (long long)sequence, (long long)batch);
  if (position >= max_tokens_per_sequence)
    return fail(VPA_ERR_INVALID_ARGUMENT,
                "%s: position exceeds paged kv cache capacity: position=%lld "
                "max_tokens_per_sequence=%lld",
                op, (long long)position, (long long)max_tokens_per_sequence);
  *slot = sequence * blocks_per_sequence * block_size + position;
  return VPA_OK;
}

int32_t vpa_graph_batch_bucket(int32_t actual_batch, int32_t max_batch) {
  if (actual_batch <= 0 || max_batch <= 0 || actual_batch > max_batch) return 0;
  int32_t bucket;
  if (actual_batch <= 2) bucket = actual_batch;
  else if (actual_batch <= 4) bucket = 4;
  else if (actual_batch <= 8) bucket = 8;
  else bucket = (int32_t)div_ceil(actual_batch, 16) * 16;
  return std::min(bucket, max_batch);
}

int vpa_graph_batch_buckets(int32_t max_batch, int32_t* buckets, int32_t capacity,
                            int32_t* count) {
  clear_error();
  if (count == nullptr || capacity < 0 || (buckets == nullptr && capacity > 0))
    return fail(VPA_ERR_INVALID_ARGUMENT, "graph_batch_buckets: bad arguments");
  const int32_t limit = std::min(std::max(max_batch, 0), kGraphMaxBatch);
  std::vector<int32_t> out;
  if (limit > 0) {
    for (int32_t b : {1, 2, 4, 8})
      if (b <= limit) out.push_back(b);
    for (int32_t b = 16; b <= limit; b += 16) out.push_back(b);
    if (out.back() != limit) out.push_back(limit);
  }
  *count = (int32_t)out.size();
  if ((int32_t)out.size() > capacity)
    return fail(VPA_ERR_CAPACITY, "graph_batch_buckets: %zu buckets, capacity %d", out.size(),
                capacity);
  std::copy(out.begin(), out.end(), buckets);
  return VPA_OK;
}

int64_t vpa_bucket_block_table_cols(int64_t blocks, int32_t block_size) {
  if (block_size <= 0) return 0;
  const int64_t block_bucket = std::max<int64_t>(div_ceil(kGraphContextBucketTokens, block_size), 1);
  if (blocks <= 0) return block_bucket;
  int64_t p = 1;
  while (p < blocks) p <<= 1;
  return std::max(p, block_bucket);
}

int vpa_pad_decode_batch(int32_t max_batch, int32_t actual_batch, const uint32_t* input_ids,
                         const int64_t* slots, const uint32_t* context_lens,
                         const uint32_t* block_tables, int32_t cols_in, int32_t cols_out,
                         uint32_t* out_input_ids, int64_t* out_slots,
                         uint32_t* out_context_lens, uint32_t* out_block_tables) {
  clear_error();
  const char* op = "pad_decode_batch";
  if (actual_batch <= 0 || actual_batch > max_batch)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: actual batch %d exceeds cuda graph max batch %d",
                op, actual_batch, max_batch);
  if (cols_in < 0 || cols_out < cols_in)
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: cannot pad block tables from %d columns down to %d",
                op, cols_in, cols_out);
  if (slots == nullptr || context_lens == nullptr || out_slots == nullptr ||
      out_context_lens == nullptr || out_block_tables == nullptr ||
      (block_tables == nullptr && cols_in > 0) ||
      (out_input_ids != nullptr && input_ids == nullptr))
    return fail(VPA_ERR_INVALID_ARGUMENT, "%s: bad arguments", op);
  for (int32_t r = 0; r < max_batch; ++r) {
    uint32_t* row = out_block_tables + (int64_t)r * cols_out;
    if (r < actual_batch) {
      if (out_input_ids != nullptr) out_input_ids[r] = input_ids[r];
      out_slots[r] = slots[r];
      out_context_lens[r] = context_lens[r];
      const uint32_t* in = block_tables + (int64_t)r * cols_in;
      for (int32_t c = 0; c < cols_out; ++c)
        row[c] = cols_in == 0 ? 0u : in[std::min(c, cols_in - 1)];
    } else {
      if (out_input_ids != nullptr) out_input_ids[r] = 0u;
      out_slots[r] = 0;
      out_context_lens[r] = 1u;
      for (int32_t c = 0; c < cols_out; ++c) row[c] = 0u;
    }
  }
  return VPA_OK;
}

}  // extern "C"
