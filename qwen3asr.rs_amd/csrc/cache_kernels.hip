// Paged-cache data movement for gfx950: reshape_and_cache (append new K/V
// rows at slot_mapping) and gather_kv_cache (paged -> packed rows).
//
// Layout (vasr-paged-attn/src/paged_kv_cache.rs:263-294, inverse restated at
// vasr-models/src/model/generation.rs:338-440):
//   key tile   of (block, head): [head_dim / x][block_size][x]
//   value tile of (block, head): [head_dim][block_size]
// Both tiles are head_dim*block_size contiguous elements.
//
// Both kernels work on one (group of block_size tokens, kv head) per
// workgroup and stage the rows in LDS, so that HBM reads and writes are
// 16-byte vectors laid out consecutively along the token axis. When a group's
// slots fill exactly one whole block (the prefill case) the workgroup writes
// the two 4 KiB (bf16) tiles as straight contiguous vectors.
//
// A workgroup whose tokens each sit alone in their cache block (a decode
// append: one new token per sequence) writes with non-temporal stores.
// It changes one 2-byte value per value-tile row, so a decode step leaves
// hundreds of thousands of partially written sectors; written back through
// L2 they slowed the decode launched right after the append by ~13 us per
// layer (c3), streamed out with the stores themselves they cost nothing
// later. Tokens that share blocks (prefill runs) fill whole sectors together
// and use ordinary stores, which are faster for them.

#include <type_traits>

#include "vpa_device.h"
#include "vpa_internal.h"

namespace vpa {
namespace {

constexpr int kThreads = 256;

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void store_stream(uint4* dst, const uint4& v) {
  __builtin_nontemporal_store(u32x4_t{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4_t*>(dst));
}
template <typename T>
__device__ __forceinline__ void store_stream(T* dst, T v) {
  static_assert(sizeof(T) == 2 || sizeof(T) == 4, "cache element");
  if constexpr (sizeof(T) == 2)
    __builtin_nontemporal_store(__builtin_bit_cast(unsigned short, v),
                                reinterpret_cast<unsigned short*>(dst));
  else
    __builtin_nontemporal_store(__builtin_bit_cast(unsigned int, v),
                                reinterpret_cast<unsigned int*>(dst));
}

template <typename T, int D, int BS>
__global__ __launch_bounds__(kThreads) void reshape_and_cache_kernel(
    const T* __restrict__ key, const T* __restrict__ value, int64_t key_token_stride,
    int64_t value_token_stride, T* __restrict__ key_cache, T* __restrict__ value_cache,
    const int64_t* __restrict__ slot_mapping, int64_t num_tokens, int64_t num_slots,
    int64_t block_stride, int64_t head_stride) {
  constexpr int X = pack_x<T>();
  constexpr int CH = D / X;       // 16-byte chunks per row
  constexpr int NV = CH * BS;     // 16-byte vectors per tile
  constexpr int VR = BS / X;      // 16-byte vectors per value-tile row (may be 0)
  static_assert(D % X == 0, "head_dim must be a multiple of x");

  __shared__ uint4 k_rows[NV];  // [token][chunk]
  __shared__ uint4 v_rows[NV];  // [token][chunk]
  __shared__ int64_t slots[BS];

  const int tid = threadIdx.x;
  const int head = blockIdx.y;
  const int64_t t0 = (int64_t)blockIdx.x * BS;

  if (tid < BS) {
    const int64_t t = t0 + tid;
    int64_t s = t < num_tokens ? slot_mapping[t] : -1;
    if (s >= num_slots) s = -1;  // out-of-range slots are skipped like padding
    slots[tid] = s;
  }
  for (int i = tid; i < NV; i += kThreads) {
    const int t = i / CH;
    const int c = i - t * CH;
    const int64_t tok = t0 + t;
    if (tok < num_tokens) {
      k_rows[i] = *reinterpret_cast<const uint4*>(key + tok * key_token_stride +
                                                  (int64_t)head * D + c * X);
      v_rows[i] = *reinterpret_cast<const uint4*>(value + tok * value_token_stride +
                                                  (int64_t)head * D + c * X);
    }
  }
  __syncthreads();

  const int64_t s0 = slots[0];
  bool whole_block = s0 >= 0 && (s0 % BS) == 0;
#pragma unroll
  for (int i = 1; i < BS; ++i) whole_block = whole_block && (slots[i] == s0 + i);

  if (whole_block && VR > 0) {
    const int64_t blk = s0 / BS;
    uint4* kt = reinterpret_cast<uint4*>(key_cache + blk * block_stride + head * head_stride);
    uint4* vt = reinterpret_cast<uint4*>(value_cache + blk * block_stride + head * head_stride);
    const T* vsrc = reinterpret_cast<const T*>(v_rows);
    for (int i = tid; i < NV; i += kThreads) {
      // key tile vector i = (chunk c, offset t)
      const int c = i / BS;
      const int t = i - c * BS;
      kt[i] = k_rows[t * CH + c];
      // value tile vector i = (dim d, token segment sg): tokens sg*X .. sg*X+X-1
      const int d = i / (VR > 0 ? VR : 1);
      const int sg = i - d * (VR > 0 ? VR : 1);
      union {
        uint4 v;
        T e[X];
      } u;
#pragma unroll
      for (int e = 0; e < X; ++e) u.e[e] = vsrc[(sg * X + e) * D + d];
      vt[i] = u.v;
    }
    return;
  }

  // General path: arbitrary slot per token. Lanes run along the token axis so
  // that tokens sharing a block still produce adjacent addresses.
  bool all_alone = true;  // no two tokens of the workgroup share a block
#pragma unroll
  for (int i = 1; i < BS; ++i)
    all_alone = all_alone && !(slots[i] >= 0 && slots[i - 1] >= 0 &&
                               slots[i] / BS == slots[i - 1] / BS);
  auto write_tokens = [&](auto streaming) {
    for (int i = tid; i < NV; i += kThreads) {
      const int c = i / BS;
      const int t = i - c * BS;
      const int64_t s = slots[t];
      if (s >= 0) {
        const int64_t blk = s / BS;
        const int off = (int)(s - blk * BS);
        uint4* dst = reinterpret_cast<uint4*>(key_cache + blk * block_stride +
                                              head * head_stride + (int64_t)(c * BS + off) * X);
        if constexpr (decltype(streaming)::value) store_stream(dst, k_rows[t * CH + c]);
        else *dst = k_rows[t * CH + c];
      }
    }
    const T* vsrc = reinterpret_cast<const T*>(v_rows);
    for (int i = tid; i < D * BS; i += kThreads) {
      const int d = i / BS;
      const int t = i - d * BS;
      const int64_t s = slots[t];
      if (s >= 0) {
        const int64_t blk = s / BS;
        const int off = (int)(s - blk * BS);
        T* dst = &value_cache[blk * block_stride + head * head_stride + (int64_t)d * BS + off];
        if constexpr (decltype(streaming)::value) store_stream(dst, vsrc[t * D + d]);
        else *dst = vsrc[t * D + d];
      }
    }
  };
  if (all_alone) write_tokens(std::true_type{});  // uniform over the workgroup
  else write_tokens(std::false_type{});
}

// One workgroup per (block column b of sequence s, kv head): copies tokens
// b*BS .. min(b*BS+BS, kv_len) of that sequence into packed rows.
template <typename T, int D, int BS>
__global__ __launch_bounds__(kThreads) void gather_kv_cache_kernel(
    T* __restrict__ out_key, T* __restrict__ out_value, const T* __restrict__ key_cache,
    const T* __restrict__ value_cache, const uint32_t* __restrict__ block_tables,
    int32_t block_table_stride, const uint32_t* __restrict__ cu_seqlens, int64_t num_blocks,
    int64_t block_stride, int64_t head_stride, int32_t num_kv_heads) {
  constexpr int X = pack_x<T>();
  constexpr int CH = D / X;
  constexpr int NV = CH * BS;

  __shared__ uint4 k_tile[NV];
  __shared__ T v_tile[D * BS];

  const int tid = threadIdx.x;
  const int b = blockIdx.x;
  const int s = blockIdx.y;
  const int head = blockIdx.z;
  const uint32_t row0 = cu_seqlens[s];
  const int64_t kv_len = (int64_t)cu_seqlens[s + 1] - (int64_t)row0;
  const int64_t tok0 = (int64_t)b * BS;
  if (tok0 >= kv_len) return;
  const int ntok = (int)min((int64_t)BS, kv_len - tok0);
  const uint32_t phys = block_tables[(int64_t)s * block_table_stride + b];
  const bool valid = (int64_t)phys < num_blocks;

  if (valid) {
    const uint4* kt =
        reinterpret_cast<const uint4*>(key_cache + (int64_t)phys * block_stride + head * head_stride);
    const uint4* vt = reinterpret_cast<const uint4*>(value_cache + (int64_t)phys * block_stride +
                                                     head * head_stride);
    uint4* vdst = reinterpret_cast<uint4*>(v_tile);
    for (int i = tid; i < NV; i += kThreads) {
      k_tile[i] = kt[i];
      vdst[i] = vt[i];
    }
  }
  __syncthreads();

  const int64_t row_stride = (int64_t)num_kv_heads * D;
  // key rows: vector (t, c) <- key tile vector (c, t)
  for (int i = tid; i < NV; i += kThreads) {
    const int t = i / CH;
    const int c = i - t * CH;
    if (t < ntok) {
      uint4 v = valid ? k_tile[c * BS + t] : make_uint4(0, 0, 0, 0);
      *reinterpret_cast<uint4*>(out_key + ((int64_t)row0 + tok0 + t) * row_stride +
                                (int64_t)head * D + c * X) = v;
    }
  }
  // value rows: vector (t, c) gathers X dims of token t from the [D][BS] tile
  for (int i = tid; i < NV; i += kThreads) {
    const int t = i / CH;
    const int c = i - t * CH;
    if (t < ntok) {
      union {
        uint4 v;
        T e[X];
      } u;
      if (valid) {
#pragma unroll
        for (int e = 0; e < X; ++e) u.e[e] = v_tile[(c * X + e) * BS + t];
      } else {
        u.v = make_uint4(0, 0, 0, 0);
      }
      *reinterpret_cast<uint4*>(out_value + ((int64_t)row0 + tok0 + t) * row_stride +
                                (int64_t)head * D + c * X) = u.v;
    }
  }
}

template <typename T, int D, int BS>
hipError_t launch_rc(const void* key, const void* value, int64_t kts, int64_t vts, void* kc,
                     void* vc, const int64_t* slots, int64_t num_tokens, const CacheGeom& g,
                     hipStream_t stream) {
  const int64_t groups = (num_tokens + BS - 1) / BS;
  dim3 grid((unsigned)groups, (unsigned)g.num_kv_heads);
  hipLaunchKernelGGL((reshape_and_cache_kernel<T, D, BS>), grid, dim3(kThreads), 0, stream,
                     static_cast<const T*>(key), static_cast<const T*>(value), kts, vts,
                     static_cast<T*>(kc), static_cast<T*>(vc), slots, num_tokens,
                     g.num_blocks * (int64_t)BS, g.block_stride, g.head_stride);
  return hipGetLastError();
}

template <typename T, int D, int BS>
hipError_t launch_gather(void* ok, void* ov, const void* kc, const void* vc,
                         const uint32_t* bt, int32_t bts, const uint32_t* cu, int32_t num_seqs,
                         const CacheGeom& g, hipStream_t stream) {
  dim3 grid((unsigned)bts, (unsigned)num_seqs, (unsigned)g.num_kv_heads);
  hipLaunchKernelGGL((gather_kv_cache_kernel<T, D, BS>), grid, dim3(kThreads), 0, stream,
                     static_cast<T*>(ok), static_cast<T*>(ov), static_cast<const T*>(kc),
                     static_cast<const T*>(vc), bt, bts, cu, g.num_blocks, g.block_stride,
                     g.head_stride, g.num_kv_heads);
  return hipGetLastError();
}

// Dispatch over the compiled (dtype, head_dim, block_size) set.
template <template <typename, int, int> class F, typename... A>
hipError_t dispatch_cache(int dtype, int D, int BS, A&&... args);

#define VPA_CACHE_CASES(FN, T)                          \
  if (D == 64 && BS == 8) return FN<T, 64, 8>(args...);   \
  if (D == 64 && BS == 16) return FN<T, 64, 16>(args...); \
  if (D == 64 && BS == 32) return FN<T, 64, 32>(args...); \
  if (D == 128 && BS == 8) return FN<T, 128, 8>(args...); \
  if (D == 128 && BS == 16) return FN<T, 128, 16>(args...); \
  if (D == 128 && BS == 32) return FN<T, 128, 32>(args...); \
  if (D == 256 && BS == 8) return FN<T, 256, 8>(args...); \
  if (D == 256 && BS == 16) return FN<T, 256, 16>(args...); \
  if (D == 256 && BS == 32) return FN<T, 256, 32>(args...);

template <typename... A>
hipError_t dispatch_rc(int dtype, int D, int BS, A... args) {
  if (dtype == VPA_DTYPE_F32) { VPA_CACHE_CASES(launch_rc, float) }
  if (dtype == VPA_DTYPE_BF16) { VPA_CACHE_CASES(launch_rc, bf16_t) }
  if (dtype == VPA_DTYPE_F16) { VPA_CACHE_CASES(launch_rc, f16_t) }
  return hipErrorInvalidValue;
}

template <typename... A>
hipError_t dispatch_gather(int dtype, int D, int BS, A... args) {
  if (dtype == VPA_DTYPE_F32) { VPA_CACHE_CASES(launch_gather, float) }
  if (dtype == VPA_DTYPE_BF16) { VPA_CACHE_CASES(launch_gather, bf16_t) }
  if (dtype == VPA_DTYPE_F16) { VPA_CACHE_CASES(launch_gather, f16_t) }
  return hipErrorInvalidValue;
}

}  // namespace

bool cache_kernels_supported(int dtype, int head_dim, int block_size) {
  const bool dt = dtype == VPA_DTYPE_F32 || dtype == VPA_DTYPE_BF16 || dtype == VPA_DTYPE_F16;
  const bool d = head_dim == 64 || head_dim == 128 || head_dim == 256;
  const bool bs = block_size == 8 || block_size == 16 || block_size == 32;
  return dt && d && bs;
}

hipError_t launch_reshape_and_cache(int dtype, const void* key, const void* value,
                                    int64_t key_token_stride, int64_t value_token_stride,
                                    void* key_cache, void* value_cache,
                                    const int64_t* slot_mapping, int64_t num_tokens,
                                    const CacheGeom& g, hipStream_t stream) {
  return dispatch_rc(dtype, g.head_dim, g.block_size, key, value, key_token_stride,
                     value_token_stride, key_cache, value_cache, slot_mapping, num_tokens, g,
                     stream);
}

hipError_t launch_gather_kv_cache(int dtype, void* out_key, void* out_value,
                                  const void* key_cache, const void* value_cache,
                                  const uint32_t* block_tables, int32_t block_table_stride,
                                  const uint32_t* cu_seqlens, int32_t num_seqs,
                                  const CacheGeom& g, hipStream_t stream) {
  return dispatch_gather(dtype, g.head_dim, g.block_size, out_key, out_value, key_cache,
                         value_cache, block_tables, block_table_stride, cu_seqlens, num_seqs,
                         g, stream);
}

}  // namespace vpa
