// Paged-attention decode for gfx950: one wavefront per (kv head, sequence,
// split-K partition of kDecodePartitionTokens tokens), serving all the query
// heads of that kv head (GQA), plus a reduce kernel that merges partitions.
//
// Semantics follow the reference's decode call
// (vasr-models/src/model/thinker_text.rs:1126-1139) with the eager attention
// it stands in for (vasr-models/src/model/attention.rs:12-21, 243-286): for
// query head h, kv head j = h / G,
//   out = sum_t exp(s_t - m) V_t / (sum_t exp(s_t - m) + 1e-6),
//   s_t = scale * q . K_t, t < context_len,
// with the +1e-6 in the denominator as in the paged kernels' sibling
// (vasr-paged-attn/src/metal/kernels/prefill_paged_attn.metal:1300).
//
// Work per wave and partition (two passes over the partition's blocks):
//   K pass: each lane loads 16-byte vectors lane + 64k of the (block, head)
//     key tile [D/x][BS][x]; that lane then owns token lane % BS and chunks
//     lane / BS + k * (64 / BS). Partial dot products are summed across the
//     64 / BS lanes of a token, the logits go to LDS.
//   softmax: max and exp-sum over the partition's logits in LDS.
//   V pass: each lane loads 16-byte vectors lane + 64k of the value tile
//     [D][BS]; that lane owns dims lane / (BS/x) + k * 64 / (BS/x) and
//     tokens (lane % (BS/x)) * x .. + x - 1, reading their probabilities
//     from LDS.
// Every HBM access is a whole 1 KiB wave-wide run of 16-byte vectors.

#include <math.h>

#include "vpa_device.h"
#include "vpa_internal.h"

namespace vpa {
namespace {

constexpr int kPT = kDecodePartitionTokens;

template <typename T, int D, int BS, int G>
__global__ __launch_bounds__(64) void paged_decode_kernel(
    T* __restrict__ out, const T* __restrict__ query, const T* __restrict__ key_cache,
    const T* __restrict__ value_cache, const uint32_t* __restrict__ block_tables,
    int32_t block_table_stride, const uint32_t* __restrict__ context_lens, int32_t max_ctx,
    float scale, int32_t num_heads, int64_t num_blocks, int64_t block_stride,
    int64_t head_stride, float* __restrict__ part_out, float* __restrict__ part_max,
    float* __restrict__ part_sum, int32_t max_parts) {
  constexpr int X = pack_x<T>();
  constexpr int LPT = 64 / BS;          // lanes per token in the key tile
  constexpr int KPL = D * BS / X / 64;  // key (and value) vectors per lane per block
  constexpr int VR = BS / X;            // vectors per value-tile row
  constexpr int DSTEP = 64 / VR;        // dim stride between a lane's value rows
  constexpr int PB = kPT / BS;          // blocks per partition
  // Blocks whose loads are issued together: 16 vectors (64 VGPRs) in flight.
  constexpr int kUnroll = KPL >= 16 ? 1 : (16 / KPL > 4 ? 4 : 16 / KPL);
  static_assert(KPL >= 1 && (D * BS / X) % 64 == 0, "tile must cover the wave");
  static_assert(PB <= 64, "block-table slice must fit one wave");

  __shared__ float s_p[G][kPT];

  const int lane = threadIdx.x;
  const int j = blockIdx.x;  // kv head
  const int s = blockIdx.y;  // sequence
  const int part = blockIdx.z;

  const int L = min((int)min(context_lens[s], (uint32_t)max_ctx), block_table_stride * BS);
  const int nblk = (L + BS - 1) / BS;
  const int nparts = (nblk + PB - 1) / PB;

  if (L <= 0) {
    // empty context: zeros (one partition writes them)
    if (part == 0) {
      for (int g = 0; g < G; ++g)
        for (int d = lane; d < D; d += 64)
          store_from_f32<T>(out + ((int64_t)s * num_heads + j * G + g) * D + d, 0.f);
    }
    return;
  }
  if (part >= nparts) return;

  const int b_begin = part * PB;
  const int b_end = min(b_begin + PB, nblk);
  const int nb = b_end - b_begin;
  const uint32_t* bt_row = block_tables + (int64_t)s * block_table_stride;
  const uint32_t my_bt = lane < nb ? bt_row[b_begin + lane] : 0u;

  // Query chunks this lane multiplies against in the key tile.
  uint4 qv[G][KPL];
  {
    const int c0 = lane / BS;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const T* qrow = query + ((int64_t)s * num_heads + j * G + g) * D;
#pragma unroll
      for (int k = 0; k < KPL; ++k)
        qv[g][k] = *reinterpret_cast<const uint4*>(qrow + (c0 + k * LPT) * X);
    }
  }

  const int64_t head_off = (int64_t)j * head_stride;
  const uint4* kbase = reinterpret_cast<const uint4*>(key_cache + head_off);
  const uint4* vbase = reinterpret_cast<const uint4*>(value_cache + head_off);
  const int64_t bstride_v = block_stride / X;  // block stride in 16-byte vectors
  const int my_tok = lane % BS;

  // ---- K pass: logits of this partition into LDS ----
  for (int b = 0; b < nb; b += kUnroll) {
    uint4 kv[kUnroll][KPL];
    bool ok[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int bi = b + u;
      const uint32_t phys = (uint32_t)__builtin_amdgcn_readlane((int)my_bt, bi < nb ? bi : 0);
      ok[u] = bi < nb && (int64_t)phys < num_blocks;
      const uint4* kp = kbase + (int64_t)(ok[u] ? phys : 0u) * bstride_v;
#pragma unroll
      for (int k = 0; k < KPL; ++k) kv[u][k] = ok[u] ? kp[lane + 64 * k] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int bi = b + u;
      if (bi < nb) {
        const int tok = (b_begin + bi) * BS + my_tok;
        const bool valid = ok[u] && tok < L;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float acc = 0.f;
#pragma unroll
          for (int k = 0; k < KPL; ++k) acc = dot16<T>(qv[g][k], kv[u][k], acc);
          acc = wave_sum_range<BS, 32>(acc);
          const float logit = valid ? acc * scale : -INFINITY;
          if (lane < BS) s_p[g][bi * BS + lane] = logit;
        }
      }
    }
  }
  lds_wave_sync();

  // ---- softmax over the partition ----
  const int ntok = nb * BS;
  float m[G], lsum[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float mx = -INFINITY;
    for (int i = lane; i < ntok; i += 64) mx = fmaxf(mx, s_p[g][i]);
    mx = wave_max_range<1, 32>(mx);
    float sm = 0.f;
    for (int i = lane; i < ntok; i += 64) {
      const float lg = s_p[g][i];
      const float p = lg == -INFINITY ? 0.f : expf(lg - mx);
      s_p[g][i] = p;
      sm += p;
    }
    m[g] = mx;
    lsum[g] = wave_sum_range<1, 32>(sm);
  }
  lds_wave_sync();

  // ---- V pass ----
  const int seg = lane % VR;
  float acc[G][KPL];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int k = 0; k < KPL; ++k) acc[g][k] = 0.f;

  for (int b = 0; b < nb; b += kUnroll) {
    uint4 vv[kUnroll][KPL];
    bool ok[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int bi = b + u;
      const uint32_t phys = (uint32_t)__builtin_amdgcn_readlane((int)my_bt, bi < nb ? bi : 0);
      ok[u] = bi < nb && (int64_t)phys < num_blocks;
      const uint4* vp = vbase + (int64_t)(ok[u] ? phys : 0u) * bstride_v;
#pragma unroll
      for (int k = 0; k < KPL; ++k) vv[u][k] = ok[u] ? vp[lane + 64 * k] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int bi = b + u;
      if (bi < nb && ok[u]) {
        const int tok0 = (b_begin + bi) * BS + seg * X;  // first token of this lane's segment
        // Tokens past the context in the last block: zero the values so stale
        // cache contents (even NaN bit patterns) cannot leak in.
        if (tok0 + X > L) {
#pragma unroll
          for (int k = 0; k < KPL; ++k) {
            union {
              uint4 v;
              T e[X];
            } w;
            w.v = vv[u][k];
#pragma unroll
            for (int e = 0; e < X; ++e)
              if (tok0 + e >= L) w.e[e] = T{};
            vv[u][k] = w.v;
          }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float* pp = &s_p[g][bi * BS + seg * X];
          if constexpr (X == 4) {
            const float4 p4 = *reinterpret_cast<const float4*>(pp);
#pragma unroll
            for (int k = 0; k < KPL; ++k) {
              const uint4 v = vv[u][k];
              float a = acc[g][k];
              a = fmaf(p4.x, __uint_as_float(v.x), a);
              a = fmaf(p4.y, __uint_as_float(v.y), a);
              a = fmaf(p4.z, __uint_as_float(v.z), a);
              a = fmaf(p4.w, __uint_as_float(v.w), a);
              acc[g][k] = a;
            }
          } else {
            // 16-bit caches: probabilities rounded to the cache type, pairs
            // of tokens per v_dot2.
            const float4 pa = *reinterpret_cast<const float4*>(pp);
            const float4 pb = *reinterpret_cast<const float4*>(pp + 4);
            const uint4 pk = make_uint4(pack2<T>(pa.x, pa.y), pack2<T>(pa.z, pa.w),
                                        pack2<T>(pb.x, pb.y), pack2<T>(pb.z, pb.w));
#pragma unroll
            for (int k = 0; k < KPL; ++k) acc[g][k] = dot16<T>(pk, vv[u][k], acc[g][k]);
          }
        }
      }
    }
  }

  // combine the VR lanes that share a dim
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int k = 0; k < KPL; ++k) {
      if constexpr (VR > 1) acc[g][k] = wave_sum_range<1, VR / 2>(acc[g][k]);
    }

  const int dim0 = lane / VR;
  if (nparts == 1) {
    if (seg == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float inv = 1.f / (lsum[g] + 1e-6f);
        T* orow = out + ((int64_t)s * num_heads + j * G + g) * D;
#pragma unroll
        for (int k = 0; k < KPL; ++k) store_from_f32<T>(orow + dim0 + k * DSTEP, acc[g][k] * inv);
      }
    }
  } else {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int64_t row = ((int64_t)s * num_heads + j * G + g) * max_parts + part;
      if (seg == 0) {
#pragma unroll
        for (int k = 0; k < KPL; ++k) part_out[row * D + dim0 + k * DSTEP] = acc[g][k];
      }
      if (lane == 0) {
        part_max[row] = m[g];
        part_sum[row] = lsum[g];
      }
    }
  }
}

// One wave per (query head, sequence) with more than one partition.
template <typename T, int D>
__global__ __launch_bounds__(64) void paged_decode_reduce_kernel(
    T* __restrict__ out, const uint32_t* __restrict__ context_lens, int32_t max_ctx,
    int32_t block_table_stride, int32_t block_size, int32_t num_heads,
    const float* __restrict__ part_out, const float* __restrict__ part_max,
    const float* __restrict__ part_sum, int32_t max_parts) {
  __shared__ float s_w[kDecodeMaxPartitions];
  const int lane = threadIdx.x;
  const int h = blockIdx.x;
  const int s = blockIdx.y;
  const int L = min((int)min(context_lens[s], (uint32_t)max_ctx), block_table_stride * block_size);
  const int nparts = (L + kPT - 1) / kPT;
  if (nparts <= 1) return;

  const int64_t row0 = ((int64_t)s * num_heads + h) * max_parts;
  float mx = -INFINITY;
  for (int p = lane; p < nparts; p += 64) mx = fmaxf(mx, part_max[row0 + p]);
  mx = wave_max_range<1, 32>(mx);
  float tot = 0.f;
  for (int p = lane; p < nparts; p += 64) {
    const float pm = part_max[row0 + p];
    const float w = pm == -INFINITY ? 0.f : expf(pm - mx);
    s_w[p] = w;
    tot += w * part_sum[row0 + p];
  }
  tot = wave_sum_range<1, 32>(tot);
  lds_wave_sync();
  const float inv = 1.f / (tot + 1e-6f);
  T* orow = out + ((int64_t)s * num_heads + h) * D;
  for (int d = lane; d < D; d += 64) {
    float a = 0.f;
    for (int p = 0; p < nparts; ++p) a = fmaf(s_w[p], part_out[(row0 + p) * D + d], a);
    store_from_f32<T>(orow + d, a * inv);
  }
}

template <typename T, int D, int BS, int G>
hipError_t launch_decode_t(void* out, const void* q, const void* kc, const void* vc,
                           const uint32_t* bt, int32_t bts, const uint32_t* cl, int32_t max_ctx,
                           float scale, int32_t num_seqs, int32_t num_heads, const CacheGeom& g,
                           const DecodeWorkspace& ws, hipStream_t stream) {
  const int max_parts = (max_ctx + kPT - 1) / kPT;
  dim3 grid((unsigned)g.num_kv_heads, (unsigned)num_seqs, (unsigned)(max_parts > 0 ? max_parts : 1));
  hipLaunchKernelGGL((paged_decode_kernel<T, D, BS, G>), grid, dim3(64), 0, stream,
                     static_cast<T*>(out), static_cast<const T*>(q), static_cast<const T*>(kc),
                     static_cast<const T*>(vc), bt, bts, cl, max_ctx, scale, num_heads,
                     g.num_blocks, g.block_stride, g.head_stride, ws.part_out, ws.part_max,
                     ws.part_sum, ws.max_parts);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || max_parts <= 1) return e;
  dim3 rgrid((unsigned)num_heads, (unsigned)num_seqs);
  hipLaunchKernelGGL((paged_decode_reduce_kernel<T, D>), rgrid, dim3(64), 0, stream,
                     static_cast<T*>(out), cl, max_ctx, bts, g.block_size, num_heads, ws.part_out,
                     ws.part_max, ws.part_sum, ws.max_parts);
  return hipGetLastError();
}

#define VPA_DECODE_G(T, D, BS)                                          \
  if (group == 1) return launch_decode_t<T, D, BS, 1>(args...);         \
  if (group == 2) return launch_decode_t<T, D, BS, 2>(args...);         \
  if (group == 4) return launch_decode_t<T, D, BS, 4>(args...);

#define VPA_DECODE_DBS(T)                                   \
  if (D == 64 && BS == 8) { VPA_DECODE_G(T, 64, 8) }        \
  if (D == 64 && BS == 16) { VPA_DECODE_G(T, 64, 16) }      \
  if (D == 64 && BS == 32) { VPA_DECODE_G(T, 64, 32) }      \
  if (D == 128 && BS == 8) { VPA_DECODE_G(T, 128, 8) }      \
  if (D == 128 && BS == 16) { VPA_DECODE_G(T, 128, 16) }    \
  if (D == 128 && BS == 32) { VPA_DECODE_G(T, 128, 32) }    \
  if (D == 256 && BS == 8) { VPA_DECODE_G(T, 256, 8) }      \
  if (D == 256 && BS == 16) { VPA_DECODE_G(T, 256, 16) }    \
  if (D == 256 && BS == 32) { VPA_DECODE_G(T, 256, 32) }

template <typename... A>
hipError_t dispatch_decode(int dtype, int D, int BS, int group, A... args) {
  if (dtype == VPA_DTYPE_BF16) { VPA_DECODE_DBS(bf16_t) }
  if (dtype == VPA_DTYPE_F16) { VPA_DECODE_DBS(f16_t) }
  if (dtype == VPA_DTYPE_F32) { VPA_DECODE_DBS(float) }
  return hipErrorInvalidValue;
}

}  // namespace

bool decode_supported(int dtype, int head_dim, int block_size, int group) {
  return cache_kernels_supported(dtype, head_dim, block_size) &&
         (group == 1 || group == 2 || group == 4);
}

size_t decode_workspace_bytes(int num_seqs, int num_heads, int head_dim, int max_context_len) {
  const int max_parts = (max_context_len + kPT - 1) / kPT;
  if (max_parts <= 1 || num_seqs <= 0 || num_heads <= 0 || head_dim <= 0) return 0;
  const size_t rows = (size_t)num_seqs * (size_t)num_heads * (size_t)max_parts;
  auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
  return up(rows * (size_t)head_dim * sizeof(float)) + 2 * up(rows * sizeof(float));
}

DecodeWorkspace carve_decode_workspace(void* base, int num_seqs, int num_heads, int head_dim,
                                       int max_context_len) {
  DecodeWorkspace ws{};
  ws.max_parts = (max_context_len + kPT - 1) / kPT;
  if (ws.max_parts <= 1) return ws;
  const size_t rows = (size_t)num_seqs * (size_t)num_heads * (size_t)ws.max_parts;
  auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
  char* p = static_cast<char*>(base);
  ws.part_out = reinterpret_cast<float*>(p);
  p += up(rows * (size_t)head_dim * sizeof(float));
  ws.part_max = reinterpret_cast<float*>(p);
  p += up(rows * sizeof(float));
  ws.part_sum = reinterpret_cast<float*>(p);
  return ws;
}

hipError_t launch_paged_decode(int dtype, void* out, const void* query, const void* key_cache,
                               const void* value_cache, const uint32_t* block_tables,
                               int32_t block_table_stride, const uint32_t* context_lens,
                               int32_t max_context_len, float scale, int32_t num_seqs,
                               int32_t num_heads, const CacheGeom& g, const DecodeWorkspace& ws,
                               hipStream_t stream) {
  const int group = num_heads / g.num_kv_heads;
  return dispatch_decode(dtype, g.head_dim, g.block_size, group, out, query, key_cache,
                         value_cache, block_tables, block_table_stride, context_lens,
                         max_context_len, scale, num_seqs, num_heads, g, ws, stream);
}

}  // namespace vpa
