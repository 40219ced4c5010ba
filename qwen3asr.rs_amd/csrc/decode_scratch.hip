// paged_attention without a caller workspace: the split-K partials, the work
// list and its header live in a static device array of this library (one
// copy per GPU, held until the process ends), so the entry point allocates
// nothing — for callers that cannot call hipMalloc (code under stream
// capture that must not allocate, tight serving loops, harnesses that forbid
// allocation).
//
// The array is laid out for the kernel the configuration runs (the rows
// kernel's 2048-token chunks for 16-bit / fp8 caches with head_dim <= 128,
// the generic kernel's 256-token partitions otherwise), which is smaller
// than the caller workspace of vpa_paged_attention (sized for any kernel).
// Nothing in it needs to start at zero: the plan launch rewrites the work
// list and its header, and every partial row the merge reads is written by
// the same call first. Every call on a GPU shares that GPU's array. Calls
// outside stream capture are ordered one after another on each GPU: each
// call's stream first waits for an event recorded after the previous call
// (whatever stream that was on), so two streams or two threads do not race
// on the array. Calls captured into a graph are not ordered by the library
// (a graph cannot wait for an event recorded outside it): replays must not
// overlap another use of the array on that GPU.

#include <atomic>
#include <mutex>

#include "vpa_internal.h"

namespace vpa {
namespace {

// VPA_NOALLOC_SCRATCH_MIB (build-time, default 64): the rows-kernel layout
// of every benchmark decode shape of this package fits 64 MiB (c3, batch 256
// with contexts up to 4000: 5.3 MB; c5, batch 1024 with contexts up to 8192:
// 42 MB). Every process that loads the library holds this much of each GPU
// it runs on, whether or not it calls the allocation-free entry point.
#ifndef VPA_NOALLOC_SCRATCH_MIB
#define VPA_NOALLOC_SCRATCH_MIB 64
#endif
static_assert(VPA_NOALLOC_SCRATCH_MIB >= 1 && VPA_NOALLOC_SCRATCH_MIB <= 4096,
              "VPA_NOALLOC_SCRATCH_MIB out of range");
constexpr size_t kScratchBytes = (size_t)VPA_NOALLOC_SCRATCH_MIB << 20;

// The library's decode scratch. In host code `scratch` names a host-side
// stand-in: its device address comes from hipGetSymbolAddress, per device.
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

// Per GPU: an event recorded after the last call outside stream capture,
// which the next call's stream waits for. It is created with the lookup of
// the scratch's address (the set-up at the first call on that GPU), so no
// later call creates anything. g_order_mu is held from a call's wait
// through its record.
std::mutex g_order_mu;
hipEvent_t g_done[kMaxDevices];
std::atomic<bool> g_done_ready[kMaxDevices];
bool g_recorded[kMaxDevices];
thread_local int t_order_dev = -1;  // the device of this thread's ordered call

// Before a call's launches: outside stream capture, take the order lock and
// make the stream wait for the previous call on this GPU.
int order_before(const char* op, void* stream) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(st, &cs);
  if (e != hipSuccess)
    return fail(VPA_ERR_HIP, "%s: hipStreamIsCapturing failed: %s", op, hipGetErrorString(e));
  t_order_dev = -1;
  if (cs != hipStreamCaptureStatusNone) return VPA_OK;  // replays ordered by the caller
  int dev = -1;
  e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return fail(VPA_ERR_HIP, "%s: hipGetDevice failed: %s", op, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(VPA_ERR_UNSUPPORTED, "%s: device ordinal %d out of range", op, dev);
  if (!g_done_ready[dev].load(std::memory_order_acquire)) return VPA_OK;  // no scratch in use
  g_order_mu.lock();
  if (g_recorded[dev]) {
    e = hipStreamWaitEvent(st, g_done[dev], 0);
    if (e != hipSuccess) {
      g_order_mu.unlock();
      return fail(VPA_ERR_HIP, "%s: hipStreamWaitEvent failed: %s", op, hipGetErrorString(e));
    }
  }
  t_order_dev = dev;
  return VPA_OK;
}

// After the launches: record this call's event and release the order lock.
int order_after(const char* op, void* stream, int rc) {
  const int dev = t_order_dev;
  if (dev < 0) return rc;  // captured
  t_order_dev = -1;
  hipError_t e = hipSuccess;
  if (rc == VPA_OK) {
    e = hipEventRecord(g_done[dev], static_cast<hipStream_t>(stream));
    if (e == hipSuccess) g_recorded[dev] = true;
  }
  g_order_mu.unlock();
  if (rc == VPA_OK && e != hipSuccess)
    return fail(VPA_ERR_HIP, "%s: ordering event failed: %s", op, hipGetErrorString(e));
  return rc;
}

// Device address of the current device's copy of `scratch`, looked up once
// per device with that device current.
int scratch_address(const char* op, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return fail(VPA_ERR_HIP, "%s: hipGetDevice failed: %s", op, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(VPA_ERR_UNSUPPORTED, "%s: device ordinal %d out of range", op, dev);
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || p == nullptr)
        return fail(VPA_ERR_HIP, "%s: hipGetSymbolAddress of the decode scratch failed: %s", op,
                    hipGetErrorString(e));
      e = hipEventCreateWithFlags(&g_done[dev], hipEventDisableTiming);
      if (e != hipSuccess)
        return fail(VPA_ERR_HIP, "%s: hipEventCreateWithFlags failed: %s", op,
                    hipGetErrorString(e));
      g_done_ready[dev].store(true, std::memory_order_release);
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return VPA_OK;
}

}  // namespace

size_t noalloc_scratch_bytes() { return kScratchBytes; }

int load_device_code(const char* op) {
  void* p = nullptr;
  return scratch_address(op, &p);
}

}  // namespace vpa

using namespace vpa;

extern "C" {

int vpa_paged_attention_noalloc(void* out, const void* query, const float* k_scale,
                                const float* v_scale, const void* key_cache,
                                const void* value_cache, const uint32_t* block_tables,
                                int32_t block_table_stride, const uint32_t* context_lens,
                                const float* alibi_slopes, int32_t max_context_len,
                                float softmax_scale, float softcapping, const float* sinks,
                                int32_t num_seqs, int32_t num_heads, int32_t num_kv_heads,
                                int32_t head_dim, int32_t block_size, int64_t num_blocks,
                                int64_t cache_block_stride, int64_t cache_head_stride,
                                int32_t dtype, int32_t cache_dtype, void* stream) {
  static const DecodeScratch kScratch{kScratchBytes, scratch_address, order_before,
                                      order_after};
  return paged_attention_impl(out, query, k_scale, v_scale, key_cache, value_cache, block_tables,
                              block_table_stride, context_lens, alibi_slopes, max_context_len,
                              softmax_scale, softcapping, sinks, num_seqs, num_heads,
                              num_kv_heads, head_dim, block_size, num_blocks,
                              cache_block_stride, cache_head_stride, dtype, cache_dtype, nullptr,
                              0, stream, false, &kScratch, "paged_attention_noalloc");
}

}  // extern "C"
