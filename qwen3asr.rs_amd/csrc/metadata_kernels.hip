// Decode-step metadata and KV block allocation kept on the GPU (gfx950).
//
// The reference builds every decode step's metadata on the host and copies
// it over: the block manager grows each running request by a block when its
// next token starts one (PagedBlockManager::allocate_slots /
// try_allocate_slots, vasr-paged-attn/src/paged_cache_runtime.rs:217-380;
// FIFO free list handed out from the front, released blocks pushed to the
// back last block first), then decode_metadata_for_batch_step
// (vasr-paged-attn/src/paged_kv_cache.rs:924-1059) turns block tables and
// prompt lengths into slot_mapping (block * BS + offset of position
// prompt_len + step), context_lens (position + 1) and the padded block
// table, and uploads them. Here the same state lives in device buffers:
// per row its block table, its block count and the position of its next
// token, and one ring of free block ids with {head, count}; a step's
// metadata and growth run in one single-workgroup launch that a captured
// decode graph can replay.
//
// Allocation order: rows in index order take blocks from the ring's head,
// which is the order the reference's step loop calls allocate_slots in
// (paged_batch_engine.rs:629-639). A row grows by at most one block per
// step (one new token); a row the ring cannot serve stalls for the step
// (try_allocate_slots returning false, paged_batch_engine.rs:209-227): its
// slot is PAD_SLOT_ID, its position does not advance, and the stall count
// is reported.

#include "vpa_device.h"
#include "vpa_internal.h"

namespace vpa {
namespace {

constexpr int kMetaThreads = 1024;

// Exclusive prefix sum of v over the workgroup; *total gets the sum.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* s_tmp,
                                                         uint32_t* total) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  uint32_t x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) s_tmp[wave] = x;
  __syncthreads();
  if (tid == 0) {
    uint32_t acc = 0;
    for (int w = 0; w < kMetaThreads / 64; ++w) {
      const uint32_t t = s_tmp[w];
      s_tmp[w] = acc;
      acc += t;
    }
    s_tmp[kMetaThreads / 64] = acc;
  }
  __syncthreads();
  const uint32_t r = x - v + s_tmp[wave];
  *total = s_tmp[kMetaThreads / 64];
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(kMetaThreads) void decode_step_metadata_kernel(
    uint32_t* __restrict__ block_tables, int32_t cols, uint32_t* __restrict__ row_blocks,
    uint32_t* __restrict__ positions, const uint8_t* __restrict__ finished,
    uint32_t* __restrict__ ring, uint32_t* __restrict__ ring_state, int32_t ring_cap,
    int32_t block_size, int64_t* __restrict__ slot_mapping, uint32_t* __restrict__ context_lens,
    uint32_t* __restrict__ status, int32_t num_rows) {
  __shared__ uint32_t s_tmp[kMetaThreads / 64 + 1];
  const int tid = threadIdx.x;
  const uint32_t head = ring_state[0];
  const uint32_t avail = ring_state[1];
  uint32_t used = 0, stalled = 0, bad = 0, max_ctx = 0;
  for (int base = 0; base < num_rows; base += kMetaThreads) {
    const int r = base + tid;
    bool live = false, grow = false;
    uint32_t pos = 0, have = 0;
    if (r < num_rows && !(finished != nullptr && finished[r])) {
      live = true;
      pos = positions[r];
      have = row_blocks[r];
      const uint32_t need = pos / (uint32_t)block_size + 1;
      if (need > (uint32_t)cols || need > have + 1) {
        live = false;  // table too narrow or more than one block missing
        ++bad;
      } else {
        grow = need > have;
      }
    }
    uint32_t total;
    const uint32_t rank = block_exclusive_scan(grow ? 1u : 0u, s_tmp, &total);
    if (r < num_rows) {
      int64_t slot = -1;
      uint32_t ctx = 0;
      if (live) {
        bool ok = true;
        if (grow) {
          const uint32_t k = used + rank;
          if (k < avail) {
            const uint32_t id = ring[(head + k) % (uint32_t)ring_cap];
            block_tables[(int64_t)r * cols + have] = id;
            row_blocks[r] = have + 1;
          } else {
            ok = false;
          }
        }
        if (ok) {
          const uint32_t bi = pos / (uint32_t)block_size;
          const uint32_t blk = block_tables[(int64_t)r * cols + bi];
          slot = (int64_t)blk * block_size + pos % (uint32_t)block_size;
          ctx = pos + 1;
          positions[r] = pos + 1;
          max_ctx = max(max_ctx, ctx);
        } else {
          ++stalled;
        }
      }
      slot_mapping[r] = slot;
      context_lens[r] = ctx == 0 ? 1u : ctx;  // PAD rows attend over one token
    }
    used += min(total, avail > used ? avail - used : 0u);
  }
  // workgroup totals of the per-thread counters
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    stalled += __shfl_xor(stalled, off, 64);
    bad += __shfl_xor(bad, off, 64);
    max_ctx = max(max_ctx, (uint32_t)__shfl_xor((int)max_ctx, off, 64));
  }
  __shared__ uint32_t s_st[kMetaThreads / 64][3];
  if ((tid & 63) == 0) {
    s_st[tid >> 6][0] = stalled;
    s_st[tid >> 6][1] = bad;
    s_st[tid >> 6][2] = max_ctx;
  }
  __syncthreads();
  if (tid == 0) {
    uint32_t a = 0, b = 0, c = 0;
    for (int w = 0; w < kMetaThreads / 64; ++w) {
      a += s_st[w][0];
      b += s_st[w][1];
      c = max(c, s_st[w][2]);
    }
    status[0] = a;
    status[1] = b;
    status[2] = c;
    ring_state[0] = (head + used) % (uint32_t)ring_cap;
    ring_state[1] = avail - used;
  }
}

// Rows in index order give back blocks keep_blocks[r] .. row_blocks[r]-1,
// last block first, to the ring's tail (trim_request_to_num_tokens /
// free_request, paged_cache_runtime.rs:330-380; block id 0, the reserved
// null block, is never returned). keep_blocks[r] >= row_blocks[r] leaves
// the row unchanged.
__global__ __launch_bounds__(kMetaThreads) void release_blocks_kernel(
    const uint32_t* __restrict__ block_tables, int32_t cols, uint32_t* __restrict__ row_blocks,
    const uint32_t* __restrict__ keep_blocks, uint32_t* __restrict__ ring,
    uint32_t* __restrict__ ring_state, int32_t ring_cap, int32_t num_rows) {
  __shared__ uint32_t s_tmp[kMetaThreads / 64 + 1];
  const int tid = threadIdx.x;
  const uint32_t head = ring_state[0];
  const uint32_t count = ring_state[1];
  uint32_t added = 0;
  for (int base = 0; base < num_rows; base += kMetaThreads) {
    const int r = base + tid;
    uint32_t have = 0, keep = 0, n = 0;
    if (r < num_rows) {
      have = min(row_blocks[r], (uint32_t)cols);
      keep = keep_blocks[r];
      for (uint32_t i = keep; i < have; ++i) n += block_tables[(int64_t)r * cols + i] != 0u;
    }
    uint32_t total;
    const uint32_t off = block_exclusive_scan(n, s_tmp, &total);
    if (r < num_rows && keep < have) {
      uint32_t tail = head + count + added + off;
      for (uint32_t i = have; i-- > keep;) {
        const uint32_t id = block_tables[(int64_t)r * cols + i];
        if (id != 0u) ring[(tail++) % (uint32_t)ring_cap] = id;
      }
      row_blocks[r] = keep;
    }
    added += total;
  }
  if (tid == 0) ring_state[1] = count + added;
}

// Grow rows, in index order, to hold target_tokens[r] tokens: each row takes
// the blocks it lacks from the ring's head if all of them are there, else it
// takes none and ok[r] = 0 (try_allocate_slots, paged_cache_runtime.rs:
// 260-300, called row by row); a row whose table is too narrow fails too.
// When all rows' missing blocks fit (admission of a batch into a pool with
// room), every row succeeds and row r takes the ring entries after those of
// the rows before it: a workgroup prefix sum, then each row copies its ids.
// Otherwise the outcome of a row depends on every row before it, and one
// thread walks the rows.
__device__ __forceinline__ uint32_t blocks_missing(const uint32_t* target_tokens,
                                                   const uint32_t* row_blocks, int r,
                                                   int32_t block_size, int32_t cols) {
  const uint32_t have = row_blocks[r];
  const uint32_t need = (target_tokens[r] + (uint32_t)block_size - 1) / (uint32_t)block_size;
  return need > have && need <= (uint32_t)cols ? need - have : 0u;
}

__global__ __launch_bounds__(kMetaThreads) void allocate_rows_kernel(
    uint32_t* __restrict__ block_tables, int32_t cols, uint32_t* __restrict__ row_blocks,
    const uint32_t* __restrict__ target_tokens, uint8_t* __restrict__ ok,
    uint32_t* __restrict__ ring, uint32_t* __restrict__ ring_state, int32_t ring_cap,
    int32_t block_size, int32_t num_rows) {
  __shared__ uint32_t s_tmp[kMetaThreads / 64 + 1];
  const int tid = threadIdx.x;
  const uint32_t head0 = ring_state[0], avail0 = ring_state[1];
  uint64_t total = 0;  // blocks all rows lack
  for (int base = 0; base < num_rows; base += kMetaThreads) {
    const int r = base + tid;
    const uint32_t more =
        r < num_rows ? blocks_missing(target_tokens, row_blocks, r, block_size, cols) : 0u;
    uint32_t chunk;
    block_exclusive_scan(more, s_tmp, &chunk);
    total += chunk;
  }
  if (total <= avail0) {  // uniform: every row gets its blocks
    uint32_t used = 0;
    for (int base = 0; base < num_rows; base += kMetaThreads) {
      const int r = base + tid;
      uint32_t more = 0, need = 0, have = 0;
      if (r < num_rows) {
        have = row_blocks[r];
        need = (target_tokens[r] + (uint32_t)block_size - 1) / (uint32_t)block_size;
        more = need > have && need <= (uint32_t)cols ? need - have : 0u;
      }
      uint32_t chunk;
      const uint32_t rank = block_exclusive_scan(more, s_tmp, &chunk);
      if (r < num_rows) {
        for (uint32_t i = 0; i < more; ++i)
          block_tables[(int64_t)r * cols + have + i] =
              ring[(head0 + used + rank + i) % (uint32_t)ring_cap];
        if (more > 0) row_blocks[r] = need;
        ok[r] = need <= (uint32_t)cols || need <= have ? 1 : 0;
      }
      used += chunk;
    }
    if (tid == 0) {
      ring_state[0] = (uint32_t)((head0 + total) % (uint32_t)ring_cap);
      ring_state[1] = avail0 - (uint32_t)total;
    }
    return;
  }
  if (tid != 0) return;
  uint32_t head = head0, avail = avail0;
  for (int r = 0; r < num_rows; ++r) {
    const uint32_t have = row_blocks[r];
    const uint32_t need = (target_tokens[r] + (uint32_t)block_size - 1) / (uint32_t)block_size;
    if (need <= have) {
      ok[r] = 1;
      continue;
    }
    const uint32_t more = need - have;
    if (more > avail || need > (uint32_t)cols) {
      ok[r] = 0;
      continue;
    }
    for (uint32_t i = 0; i < more; ++i) {
      block_tables[(int64_t)r * cols + have + i] = ring[head];
      head = (head + 1) % (uint32_t)ring_cap;
    }
    avail -= more;
    row_blocks[r] = need;
    ok[r] = 1;
  }
  ring_state[0] = head;
  ring_state[1] = avail;
}

}  // namespace

hipError_t launch_allocate_rows(uint32_t* block_tables, int32_t cols, uint32_t* row_blocks,
                                const uint32_t* target_tokens, uint8_t* ok, uint32_t* ring,
                                uint32_t* ring_state, int32_t ring_cap, int32_t block_size,
                                int32_t num_rows, hipStream_t stream) {
  hipLaunchKernelGGL(allocate_rows_kernel, dim3(1), dim3(kMetaThreads), 0, stream, block_tables,
                     cols, row_blocks, target_tokens, ok, ring, ring_state, ring_cap, block_size,
                     num_rows);
  return hipGetLastError();
}

hipError_t launch_decode_step_metadata(uint32_t* block_tables, int32_t cols,
                                       uint32_t* row_blocks, uint32_t* positions,
                                       const uint8_t* finished, uint32_t* ring,
                                       uint32_t* ring_state, int32_t ring_cap,
                                       int32_t block_size, int64_t* slot_mapping,
                                       uint32_t* context_lens, uint32_t* status,
                                       int32_t num_rows, hipStream_t stream) {
  hipLaunchKernelGGL(decode_step_metadata_kernel, dim3(1), dim3(kMetaThreads), 0, stream,
                     block_tables, cols, row_blocks, positions, finished, ring, ring_state,
                     ring_cap, block_size, slot_mapping, context_lens, status, num_rows);
  return hipGetLastError();
}

hipError_t launch_release_blocks(const uint32_t* block_tables, int32_t cols,
                                 uint32_t* row_blocks, const uint32_t* keep_blocks,
                                 uint32_t* ring, uint32_t* ring_state, int32_t ring_cap,
                                 int32_t num_rows, hipStream_t stream) {
  hipLaunchKernelGGL(release_blocks_kernel, dim3(1), dim3(kMetaThreads), 0, stream,
                     block_tables, cols, row_blocks, keep_blocks, ring, ring_state, ring_cap,
                     num_rows);
  return hipGetLastError();
}

}  // namespace vpa
