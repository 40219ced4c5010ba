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
#ifndef VPA_APPEND_HEAD_FAST
#define VPA_APPEND_HEAD_FAST 1
#endif
#ifndef VPA_GATHER_HEAD_FAST
#define VPA_GATHER_HEAD_FAST 1
#endif

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void store_stream(uint4* dst, const uint4& v) {
  __builtin_nontemporal_store(u32x4_t{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4_t*>(dst));
}
template <typename T>
__device__ __forceinline__ void store_stream(T* dst, T v) {
  static_assert(sizeof(T) == 1 || sizeof(T) == 2 || sizeof(T) == 4, "cache element");
  if constexpr (sizeof(T) == 1)
    __builtin_nontemporal_store(__builtin_bit_cast(unsigned char, v),
                                reinterpret_cast<unsigned char*>(dst));
  else if constexpr (sizeof(T) == 2)
    __builtin_nontemporal_store(__builtin_bit_cast(unsigned short, v),
                                reinterpret_cast<unsigned short*>(dst));
  else
    __builtin_nontemporal_store(__builtin_bit_cast(unsigned int, v),
                                reinterpret_cast<unsigned int*>(dst));
}

// Sixteen consecutive elements of T, each divided by `scale` and encoded as
// E4M3FN, packed into one 16-byte vector (byte e = element e).
template <typename T>
__device__ __forceinline__ uint4 quantize16(const T* src, float scale) {
  uint32_t w[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint32_t b = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) b |= fp8_from_f32(load_as_f32(src + 4 * q + e) / scale) << (8 * e);
    w[q] = b;
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// T: element type of the new rows; C: cache element type (T itself, copied
// bit-exactly, or fp8_t, quantised with *k_scale / *v_scale).
template <typename T, typename C, int D, int BS>
__global__ __launch_bounds__(kThreads) void reshape_and_cache_kernel(
    const T* __restrict__ key, const T* __restrict__ value, int64_t key_token_stride,
    int64_t value_token_stride, C* __restrict__ key_cache, C* __restrict__ value_cache,
    const int64_t* __restrict__ slot_mapping, int64_t num_tokens, int64_t num_slots,
    int64_t block_stride, int64_t head_stride, const float* __restrict__ k_scale,
    const float* __restrict__ v_scale, int32_t num_kv_heads, LastSlots last) {
  constexpr bool kQuant = !std::is_same_v<T, C>;
  static_assert(!kQuant || std::is_same_v<C, fp8_t>, "a cache type differing from the rows is fp8");
  constexpr int X = pack_x<C>();
  constexpr int CH = D / X;       // 16-byte chunks per row
  constexpr int NV = CH * BS;     // 16-byte vectors per tile
  constexpr int VR = BS / X;      // 16-byte vectors per value-tile row (may be 0)
  static_assert(D % X == 0, "head_dim must be a multiple of x");

  __shared__ uint4 k_rows[NV];  // [token][chunk]
  __shared__ uint4 v_rows[NV];  // [token][chunk]
  __shared__ int64_t slots[BS];

  const int tid = threadIdx.x;
#if VPA_APPEND_HEAD_FAST
  // kv heads vary fastest over the grid: consecutive workgroups read the
  // adjacent head slices of the same token rows and write the adjacent head
  // tiles of the same cache block
  const int head = (int)(blockIdx.x % (uint32_t)num_kv_heads);
  const int64_t t0 = (int64_t)(blockIdx.x / (uint32_t)num_kv_heads) * BS;
#else
  const int head = blockIdx.y;
  const int64_t t0 = (int64_t)blockIdx.x * BS;
#endif

  if (tid < BS) {
    const int64_t t = t0 + tid;
    int64_t s = -1;
    if (t < num_tokens) {
      if (slot_mapping != nullptr) {
        s = slot_mapping[t];
      } else {
        // row t is sequence t's token at position context_lens[t] - 1 (none
        // for an empty context or one the table or max_context_len clamps)
        const uint32_t L = last.context_lens[t];
        if (L >= 1u && L <= (uint32_t)last.cap) {
          const uint32_t pos = L - 1u;
          s = (int64_t)last.block_tables[t * (int64_t)last.stride + pos / BS] * BS + pos % BS;
        }
      }
    }
    if (s >= num_slots) s = -1;  // out-of-range slots are skipped like padding
    slots[tid] = s;
  }
  float ks = 1.f, vs = 1.f;
  if constexpr (kQuant) {
    ks = *k_scale;
    vs = *v_scale;
  }
  for (int i = tid; i < NV; i += kThreads) {
    const int t = i / CH;
    const int c = i - t * CH;
    const int64_t tok = t0 + t;
    if (tok < num_tokens) {
      const T* ksrc = key + tok * key_token_stride + (int64_t)head * D + c * X;
      const T* vsrc = value + tok * value_token_stride + (int64_t)head * D + c * X;
      if constexpr (kQuant) {
        k_rows[i] = quantize16(ksrc, ks);
        v_rows[i] = quantize16(vsrc, vs);
      } else {
        k_rows[i] = *reinterpret_cast<const uint4*>(ksrc);
        v_rows[i] = *reinterpret_cast<const uint4*>(vsrc);
      }
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
    const C* vsrc = reinterpret_cast<const C*>(v_rows);
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
        C e[X];
      } u;
#pragma unroll
      for (int e = 0; e < X; ++e) u.e[e] = vsrc[(sg * X + e) * D + d];
      vt[i] = u.v;
    }
    return;
  }

  // General path: arbitrary slot per token. Lanes run along the token axis so
  // that tokens sharing a block still produce adjacent addresses.
  // No two neighbouring tokens of the workgroup share a block (decode: one
  // token per sequence). Only neighbours are compared: tokens that share a
  // block without being adjacent (slots 5, 100, 6) also take the streaming
  // stores, which stay correct, only slower for that rare pattern.
  bool all_alone = true;
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
    const C* vsrc = reinterpret_cast<const C*>(v_rows);
    for (int i = tid; i < D * BS; i += kThreads) {
      const int d = i / BS;
      const int t = i - d * BS;
      const int64_t s = slots[t];
      if (s >= 0) {
        const int64_t blk = s / BS;
        const int off = (int)(s - blk * BS);
        C* dst = &value_cache[blk * block_stride + head * head_stride + (int64_t)d * BS + off];
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
#if VPA_GATHER_HEAD_FAST
  // kv heads fastest: consecutive workgroups read the adjacent head tiles of
  // one block and write adjacent head slices of the same rows
  const int head = blockIdx.x;
  const int b = blockIdx.y;
#else
  const int b = blockIdx.x;
  const int head = blockIdx.z;
#endif
  const int s = VPA_GATHER_HEAD_FAST ? blockIdx.z : blockIdx.y;
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
    for (int i = tid; i < NV; i += kThreads) {  // tiles are read once: streamed
      k_tile[i] = load_stream(kt + i);
      vdst[i] = load_stream(vt + i);
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

// Sixteen f32 values stored as TO (round to nearest even) with 16-byte stores.
template <typename TO>
__device__ __forceinline__ void store16(TO* dst, const float (&f)[16]) {
  uint4* d4 = reinterpret_cast<uint4*>(dst);
  if constexpr (std::is_same_v<TO, float>) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      d4[q] = make_uint4(__float_as_uint(f[4 * q]), __float_as_uint(f[4 * q + 1]),
                         __float_as_uint(f[4 * q + 2]), __float_as_uint(f[4 * q + 3]));
  } else {
    uint32_t w[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      TO lo, hi;
      store_from_f32<TO>(&lo, f[2 * q]);
      store_from_f32<TO>(&hi, f[2 * q + 1]);
      w[q] = (uint32_t)lo.x | ((uint32_t)hi.x << 16);
    }
    d4[0] = make_uint4(w[0], w[1], w[2], w[3]);
    d4[1] = make_uint4(w[4], w[5], w[6], w[7]);
  }
}

// Sixteen E4M3FN bytes -> f32 times `scale`, through the same exact
// conversion the decode kernel uses (to f16 for an f16 output, to bf16
// otherwise), then widened. The sign of each result is set last from the
// byte and the scale: the f16 path and a fused multiply-add with a +0
// addend (v_fma_mix, which the compiler picks for f16 -> f32 * s -> f16)
// both turn -0 into +0; every other value already has that sign.
template <typename TO>
__device__ __forceinline__ void fp8x16_to_f32_scaled(const uint4& v, float scale,
                                                     float (&f)[16]) {
  using P = std::conditional_t<std::is_same_v<TO, f16_t>, f16_t, bf16_t>;
  uint4 lo, hi;
  fp8x16_to_pk<P>(v, lo, hi);
  const uint32_t w[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
  const uint32_t b[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    if constexpr (std::is_same_v<P, f16_t>) {
      f[2 * q] = f16_bits_to_f32((uint16_t)(w[q] & 0xffffu));
      f[2 * q + 1] = f16_bits_to_f32((uint16_t)(w[q] >> 16));
    } else {
      f[2 * q] = bf16_bits_to_f32(w[q] & 0xffffu);
      f[2 * q + 1] = bf16_bits_to_f32(w[q] >> 16);
    }
  }
  const uint32_t sneg = __float_as_uint(scale) >> 31;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const uint32_t neg = ((b[e / 4] >> (8 * (e % 4) + 7)) & 1u) ^ sneg;
    const float m = f[e] * scale;
    f[e] = __uint_as_float((__float_as_uint(m) & 0x7fffffffu) | (neg << 31));
  }
}

// gather_kv_cache from an fp8 cache: like gather_kv_cache_kernel, each value
// dequantised as (float)byte * scale and stored as TO.
template <typename TO, int D, int BS>
__global__ __launch_bounds__(kThreads) void gather_kv_cache_fp8_kernel(
    TO* __restrict__ out_key, TO* __restrict__ out_value, const fp8_t* __restrict__ key_cache,
    const fp8_t* __restrict__ value_cache, const uint32_t* __restrict__ block_tables,
    int32_t block_table_stride, const uint32_t* __restrict__ cu_seqlens, int64_t num_blocks,
    int64_t block_stride, int64_t head_stride, int32_t num_kv_heads,
    const float* __restrict__ k_scale, const float* __restrict__ v_scale) {
  constexpr int X = 16;
  constexpr int CH = D / X;
  constexpr int NV = CH * BS;  // 16-byte vectors per tile (K and V alike)

  __shared__ uint4 k_tile[NV];
  __shared__ __align__(16) uint8_t v_tile[D * BS];

  const int tid = threadIdx.x;
#if VPA_GATHER_HEAD_FAST
  // kv heads fastest: consecutive workgroups read the adjacent head tiles of
  // one block and write adjacent head slices of the same rows
  const int head = blockIdx.x;
  const int b = blockIdx.y;
#else
  const int b = blockIdx.x;
  const int head = blockIdx.z;
#endif
  const int s = VPA_GATHER_HEAD_FAST ? blockIdx.z : blockIdx.y;
  const uint32_t row0 = cu_seqlens[s];
  const int64_t kv_len = (int64_t)cu_seqlens[s + 1] - (int64_t)row0;
  const int64_t tok0 = (int64_t)b * BS;
  if (tok0 >= kv_len) return;
  const int ntok = (int)min((int64_t)BS, kv_len - tok0);
  const uint32_t phys = block_tables[(int64_t)s * block_table_stride + b];
  const bool valid = (int64_t)phys < num_blocks;

  if (valid) {
    const int64_t off = (int64_t)phys * block_stride + head * head_stride;
    const uint4* kt = reinterpret_cast<const uint4*>(key_cache + off);
    const uint4* vt = reinterpret_cast<const uint4*>(value_cache + off);
    uint4* vdst = reinterpret_cast<uint4*>(v_tile);
    for (int i = tid; i < NV; i += kThreads) {  // tiles are read once: streamed
      k_tile[i] = load_stream(kt + i);
      vdst[i] = load_stream(vt + i);
    }
  }
  __syncthreads();
  const float ks = *k_scale, vs = *v_scale;
  const int64_t row_stride = (int64_t)num_kv_heads * D;
  for (int i = tid; i < NV; i += kThreads) {
    const int t = i / CH;
    const int c = i - t * CH;
    if (t >= ntok) continue;
    const int64_t o = ((int64_t)row0 + tok0 + t) * row_stride + (int64_t)head * D + c * X;
    float f[16];
    if (valid) {
      fp8x16_to_f32_scaled<TO>(k_tile[c * BS + t], ks, f);  // key tile vector (c, t)
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) f[e] = 0.f;
    }
    store16(out_key + o, f);
    if (valid) {
      uint32_t w[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t bword = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) bword |= (uint32_t)v_tile[(c * X + 4 * q + e) * BS + t] << (8 * e);
        w[q] = bword;
      }
      fp8x16_to_f32_scaled<TO>(make_uint4(w[0], w[1], w[2], w[3]), vs, f);
    }
    store16(out_value + o, f);
  }
}

template <typename TO, int D, int BS>
hipError_t launch_gather_fp8(void* ok, void* ov, const void* kc, const void* vc,
                             const uint32_t* bt, int32_t bts, const uint32_t* cu,
                             int32_t num_seqs, const CacheGeom& g, const float* k_scale,
                             const float* v_scale, hipStream_t stream) {
#if VPA_GATHER_HEAD_FAST
  dim3 grid((unsigned)g.num_kv_heads, (unsigned)bts, (unsigned)num_seqs);
#else
  dim3 grid((unsigned)bts, (unsigned)num_seqs, (unsigned)g.num_kv_heads);
#endif
  hipLaunchKernelGGL((gather_kv_cache_fp8_kernel<TO, D, BS>), grid, dim3(kThreads), 0, stream,
                     static_cast<TO*>(ok), static_cast<TO*>(ov), static_cast<const fp8_t*>(kc),
                     static_cast<const fp8_t*>(vc), bt, bts, cu, g.num_blocks, g.block_stride,
                     g.head_stride, g.num_kv_heads, k_scale, v_scale);
  return hipGetLastError();
}

template <typename T, typename C, int D, int BS>
hipError_t launch_rc_t(const void* key, const void* value, int64_t kts, int64_t vts, void* kc,
                       void* vc, const int64_t* slots, const LastSlots& last,
                       int64_t num_tokens, const CacheGeom& g, const float* k_scale,
                       const float* v_scale, hipStream_t stream) {
  const int64_t groups = (num_tokens + BS - 1) / BS;
#if VPA_APPEND_HEAD_FAST
  dim3 grid((unsigned)(groups * g.num_kv_heads));
#else
  dim3 grid((unsigned)groups, (unsigned)g.num_kv_heads);
#endif
  hipLaunchKernelGGL((reshape_and_cache_kernel<T, C, D, BS>), grid, dim3(kThreads), 0, stream,
                     static_cast<const T*>(key), static_cast<const T*>(value), kts, vts,
                     static_cast<C*>(kc), static_cast<C*>(vc), slots, num_tokens,
                     g.num_blocks * (int64_t)BS, g.block_stride, g.head_stride, k_scale, v_scale,
                     (int32_t)g.num_kv_heads, last);
  return hipGetLastError();
}
template <typename T, int D, int BS>
hipError_t launch_rc(const void* key, const void* value, int64_t kts, int64_t vts, void* kc,
                     void* vc, const int64_t* slots, LastSlots last, int64_t num_tokens,
                     const CacheGeom& g, const float* k_scale, const float* v_scale, bool fp8,
                     hipStream_t stream) {
  if (fp8)
    return launch_rc_t<T, fp8_t, D, BS>(key, value, kts, vts, kc, vc, slots, last, num_tokens,
                                        g, k_scale, v_scale, stream);
  return launch_rc_t<T, T, D, BS>(key, value, kts, vts, kc, vc, slots, last, num_tokens, g,
                                  k_scale, v_scale, stream);
}

template <typename T, int D, int BS>
hipError_t launch_gather(void* ok, void* ov, const void* kc, const void* vc,
                         const uint32_t* bt, int32_t bts, const uint32_t* cu, int32_t num_seqs,
                         const CacheGeom& g, hipStream_t stream) {
#if VPA_GATHER_HEAD_FAST
  dim3 grid((unsigned)g.num_kv_heads, (unsigned)bts, (unsigned)num_seqs);
#else
  dim3 grid((unsigned)bts, (unsigned)num_seqs, (unsigned)g.num_kv_heads);
#endif
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
  if (D == 96 && BS == 8) return FN<T, 96, 8>(args...);   \
  if (D == 96 && BS == 16) return FN<T, 96, 16>(args...); \
  if (D == 96 && BS == 32) return FN<T, 96, 32>(args...); \
  if (D == 192 && BS == 8) return FN<T, 192, 8>(args...); \
  if (D == 192 && BS == 16) return FN<T, 192, 16>(args...); \
  if (D == 192 && BS == 32) return FN<T, 192, 32>(args...); \
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
hipError_t dispatch_gather_fp8(int out_dtype, int D, int BS, A... args) {
  if (out_dtype == VPA_DTYPE_F32) { VPA_CACHE_CASES(launch_gather_fp8, float) }
  if (out_dtype == VPA_DTYPE_BF16) { VPA_CACHE_CASES(launch_gather_fp8, bf16_t) }
  if (out_dtype == VPA_DTYPE_F16) { VPA_CACHE_CASES(launch_gather_fp8, f16_t) }
  return hipErrorInvalidValue;
}

template <typename... A>
hipError_t dispatch_gather(int dtype, int D, int BS, A... args) {
  if (dtype == VPA_DTYPE_FP8_E4M3) { VPA_CACHE_CASES(launch_gather, fp8_t) }  // raw bytes
  if (dtype == VPA_DTYPE_F32) { VPA_CACHE_CASES(launch_gather, float) }
  if (dtype == VPA_DTYPE_BF16) { VPA_CACHE_CASES(launch_gather, bf16_t) }
  if (dtype == VPA_DTYPE_F16) { VPA_CACHE_CASES(launch_gather, f16_t) }
  return hipErrorInvalidValue;
}

}  // namespace

bool cache_kernels_supported(int dtype, int head_dim, int block_size) {
  const bool dt = dtype == VPA_DTYPE_F32 || dtype == VPA_DTYPE_BF16 ||
                  dtype == VPA_DTYPE_F16 || dtype == VPA_DTYPE_FP8_E4M3;
  const bool d = head_dim == 64 || head_dim == 96 || head_dim == 128 || head_dim == 192 ||
                 head_dim == 256;
  const bool bs = block_size == 8 || block_size == 16 || block_size == 32;
  return dt && d && bs;
}

hipError_t launch_reshape_and_cache(int dtype, int cache_dtype, const void* key,
                                    const void* value, int64_t key_token_stride,
                                    int64_t value_token_stride, void* key_cache,
                                    void* value_cache, const int64_t* slot_mapping,
                                    int64_t num_tokens, const CacheGeom& g, const float* k_scale,
                                    const float* v_scale, hipStream_t stream) {
  return dispatch_rc(dtype, g.head_dim, g.block_size, key, value, key_token_stride,
                     value_token_stride, key_cache, value_cache, slot_mapping, LastSlots{},
                     num_tokens, g, k_scale, v_scale, cache_dtype == VPA_DTYPE_FP8_E4M3, stream);
}

hipError_t launch_append_last_positions(int dtype, int cache_dtype, const void* key,
                                        const void* value, int64_t key_token_stride,
                                        int64_t value_token_stride, void* key_cache,
                                        void* value_cache, const LastSlots& last,
                                        int32_t num_seqs, const CacheGeom& g,
                                        const float* k_scale, const float* v_scale,
                                        hipStream_t stream) {
  return dispatch_rc(dtype, g.head_dim, g.block_size, key, value, key_token_stride,
                     value_token_stride, key_cache, value_cache,
                     static_cast<const int64_t*>(nullptr), last, (int64_t)num_seqs, g, k_scale,
                     v_scale, cache_dtype == VPA_DTYPE_FP8_E4M3, stream);
}

hipError_t launch_gather_kv_cache(int cache_dtype, int out_dtype, void* out_key,
                                  void* out_value, const void* key_cache,
                                  const void* value_cache, const uint32_t* block_tables,
                                  int32_t block_table_stride, const uint32_t* cu_seqlens,
                                  int32_t num_seqs, const CacheGeom& g, const float* k_scale,
                                  const float* v_scale, hipStream_t stream) {
  if (cache_dtype == VPA_DTYPE_FP8_E4M3)
    return dispatch_gather_fp8(out_dtype, g.head_dim, g.block_size, out_key, out_value,
                               key_cache, value_cache, block_tables, block_table_stride,
                               cu_seqlens, num_seqs, g, k_scale, v_scale, stream);
  return dispatch_gather(cache_dtype, g.head_dim, g.block_size, out_key, out_value, key_cache,
                         value_cache, block_tables, block_table_stride, cu_seqlens, num_seqs,
                         g, stream);
}

}  // namespace vpa
