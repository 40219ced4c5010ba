// Paged-attention decode for gfx950, two paths here:
//   * 16-bit and fp8 caches (under 16-bit queries) whose (block, head)
//     tiles are whole 1 KiB wave loads of at most 8 KiB, vASR's shapes among
//     them: a work list built on the device (decode_plan_kernel, longest
//     chunk first), paged_decode_rows_kernel (one workgroup per (chunk, kv
//     head), its waves splitting the chunk's blocks) and decode_merge_kernel
//     for the sequences longer than one chunk; described further down;
//   * f32 caches, fp8 caches under f32 queries, and the 16-bit / fp8 tiles
//     above 8 KiB (head dims 192 and 256 at 32-token blocks):
//     paged_decode_kernel, one wavefront per (kv head, sequence, split-K
//     partition of kDecodePartitionTokens tokens) serving all the query
//     heads of that kv head (GQA), and paged_decode_reduce_kernel merging
//     the partitions; described here.
// The head-dim / block-size pairs whose tiles are not whole 1 KiB loads run
// on the chunked-prefill vector kernel (prefill_vector_kernels.hip) with one
// query per sequence; api.cpp routes them.
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
// Generic path, work per wave and partition (two passes over the
// partition's blocks):
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
#include <stdlib.h>

#include <algorithm>
#include <type_traits>

#include "vpa_device.h"
#include "vpa_internal.h"

namespace vpa {
namespace {

constexpr int kPT = kDecodePartitionTokens;

#ifndef VPA_DECODE_STREAM_LOADS
#define VPA_DECODE_STREAM_LOADS 1
#endif
// K/V tile loads of the decode: every byte is read once per call, so they
// stream (non-temporal) unless VPA_DECODE_STREAM_LOADS is 0.
__device__ __forceinline__ uint4 tile_load(const uint4* p) {
  if constexpr (VPA_DECODE_STREAM_LOADS) return load_stream(p);
  else return *p;
}
// Workgroup barrier for data exchanged through LDS: waits for this wave's LDS
// operations only (outstanding global loads and stores stay in flight).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
// v with its 16-bit element e (0..7; uniform) replaced by val, without a
// runtime-indexed array
__device__ __forceinline__ uint4 put_u16(uint4 v, int e, uint32_t val) {
  const uint32_t sh = (uint32_t)(e & 1) * 16u;
  const uint32_t keep = ~(0xffffu << sh), ins = (val & 0xffffu) << sh;
  const int w = e >> 1;
  v.x = w == 0 ? (v.x & keep) | ins : v.x;
  v.y = w == 1 ? (v.y & keep) | ins : v.y;
  v.z = w == 2 ? (v.z & keep) | ins : v.z;
  v.w = w == 3 ? (v.w & keep) | ins : v.w;
  return v;
}
// 16-byte non-temporal store (the fused append's whole sectors)
__device__ __forceinline__ void tile_store(uint4* p, const uint4& v) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  __builtin_nontemporal_store(u32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4*>(p));
}

// E4M3FN byte b (0..255) of an fp8 cache as f32 (exact, through gfx950's
// conversion to bf16)
__device__ __forceinline__ float fp8_elem_f32(uint32_t b) {
  return bf16_bits_to_f32(fp8x2_to_pk<bf16_t>(b & 0xffu, false) & 0xffffu);
}

// C is the cache element type: T itself, or fp8_t (each cache element read
// as f32(E4M3FN(byte) * scale) rounded to the query type, as the reference
// dequantises; a 16-byte vector then holds 16 dims of a key or 16 tokens of
// a value row, and a lane's q chunk is 4 vectors of f32 or 2 of 16 bits).
// The fp8 instances under 16-bit queries serve the tiles the rows kernel
// does not take (head dims 192 and 256 at 32-token blocks).
template <typename T, typename C, int D, int BS, int G>
__global__ __launch_bounds__(64) void paged_decode_kernel(
    T* __restrict__ out, const T* __restrict__ query, const C* __restrict__ key_cache,
    const C* __restrict__ value_cache, const uint32_t* __restrict__ block_tables,
    int32_t block_table_stride, const uint32_t* __restrict__ context_lens, int32_t max_ctx,
    float scale, int32_t num_heads, int64_t num_blocks, int64_t block_stride,
    int64_t head_stride, float* __restrict__ part_out, float* __restrict__ part_max,
    float* __restrict__ part_sum, int32_t max_parts, int32_t kv_rep,
    const float* __restrict__ k_scale, const float* __restrict__ v_scale) {
  constexpr bool kF8 = std::is_same_v<C, fp8_t>;
  static_assert(std::is_same_v<C, T> || kF8, "cache type is the query type, or fp8");
  constexpr int X = pack_x<C>();
  constexpr int QV = X * (int)sizeof(T) / 16;  // 16-byte q vectors per key chunk
  constexpr int LPT = 64 / BS;          // lanes per token in the key tile
  constexpr int KPL = D * BS / X / 64;  // key (and value) vectors per lane per block
  constexpr int VR = BS / X;            // vectors per value-tile row
  constexpr int DSTEP = 64 / VR;        // dim stride between a lane's value rows
  constexpr int PB = kPT / BS;          // blocks per partition
  // Blocks whose loads are issued together: 16 vectors (64 VGPRs) in flight
  // (fp8: 4, whose 16 elements each are dequantised into registers)
  constexpr int kVecs = kF8 ? 4 : 16;
  constexpr int kUnroll = KPL >= kVecs ? 1 : (kVecs / KPL > 4 ? 4 : kVecs / KPL);
  static_assert(KPL >= 1 && (D * BS / X) % 64 == 0, "tile must cover the wave");
  static_assert(PB <= 64, "block-table slice must fit one wave");

  __shared__ __align__(16) float s_p[G][kPT];  // (rows read as float4 by the fp8 value pass)
  // Shapes whose query vectors would not fit registers (G x KPL x QV > 16,
  // e.g. f32 at head_dim 256 with 32-token blocks: 128 vectors per lane)
  // read them from LDS at each use instead.
  constexpr bool kQinLds = G * KPL * QV > 16;
  constexpr int CHQ = D / X;  // key chunks of a query row (QV vectors each)
  __shared__ uint4 s_q[kQinLds ? G * CHQ * QV : 1];

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

  // Query chunks this lane multiplies against in the key tile: chunk
  // lane / BS + k * LPT of each head (QV vectors each), in registers or
  // (kQinLds) in LDS.
  uint4 qv[kQinLds ? 1 : G][kQinLds ? 1 : KPL][kQinLds ? 1 : QV];
  const int c0 = lane / BS;
  if constexpr (kQinLds) {
    for (int i = lane; i < G * CHQ * QV; i += 64) {
      const int g = i / (CHQ * QV), c = i - g * (CHQ * QV);
      s_q[i] = *reinterpret_cast<const uint4*>(query + ((int64_t)s * num_heads + j * G + g) * D +
                                                c * (16 / (int)sizeof(T)));
    }
    lds_wave_sync();
  } else {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const T* qrow = query + ((int64_t)s * num_heads + j * G + g) * D;
#pragma unroll
      for (int k = 0; k < KPL; ++k)
#pragma unroll
        for (int h = 0; h < QV; ++h)
          qv[g][k][h] = *reinterpret_cast<const uint4*>(qrow + (c0 + k * LPT) * X +
                                                         h * (16 / (int)sizeof(T)));
    }
  }
  auto qchunk = [&](int g, int k, int h) -> uint4 {
    if constexpr (kQinLds) return s_q[(g * CHQ + c0 + k * LPT) * QV + h];
    else return qv[g][k][h];
  };
  const float ks = kF8 ? *k_scale : 1.f;
  const float vs = kF8 ? *v_scale : 1.f;

  // j counts kv_rep replicas of every kv head (kv_rep > 1: more query heads
  // per kv head than G), so its cache head is j / kv_rep
  const int64_t head_off = (int64_t)(j / kv_rep) * head_stride;
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
      for (int k = 0; k < KPL; ++k)
        kv[u][k] = ok[u] ? tile_load(kp + lane + 64 * k) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int bi = b + u;
      if (bi < nb) {
        const int tok = (b_begin + bi) * BS + my_tok;
        const bool valid = ok[u] && tok < L;
        // fp8: each chunk's 16 key elements dequantised once for every head
        float dots[kF8 ? G : 1];
        if constexpr (kF8) {
#pragma unroll
          for (int g = 0; g < G; ++g) dots[g] = 0.f;
#pragma unroll
          for (int k = 0; k < KPL; ++k) {
            float kf[16];
            const uint32_t w[4] = {kv[u][k].x, kv[u][k].y, kv[u][k].z, kv[u][k].w};
#pragma unroll
            for (int e = 0; e < 16; ++e) kf[e] = fp8_elem_f32(w[e / 4] >> (8 * (e % 4))) * ks;
            if constexpr (std::is_same_v<T, float>) {
#pragma unroll
              for (int g = 0; g < G; ++g)
#pragma unroll
                for (int h = 0; h < QV; ++h) {
                  const uint4 q4 = qchunk(g, k, h);
                  dots[g] = fmaf(__uint_as_float(q4.x), kf[4 * h + 0], dots[g]);
                  dots[g] = fmaf(__uint_as_float(q4.y), kf[4 * h + 1], dots[g]);
                  dots[g] = fmaf(__uint_as_float(q4.z), kf[4 * h + 2], dots[g]);
                  dots[g] = fmaf(__uint_as_float(q4.w), kf[4 * h + 3], dots[g]);
                }
            } else {
              // the elements rounded to the query type, pairs per v_dot2
              uint4 kq[2];
#pragma unroll
              for (int h = 0; h < 2; ++h)
                kq[h] = make_uint4(pack2_hw<T>(kf[8 * h + 0], kf[8 * h + 1]),
                                   pack2_hw<T>(kf[8 * h + 2], kf[8 * h + 3]),
                                   pack2_hw<T>(kf[8 * h + 4], kf[8 * h + 5]),
                                   pack2_hw<T>(kf[8 * h + 6], kf[8 * h + 7]));
#pragma unroll
              for (int g = 0; g < G; ++g)
                dots[g] = dot16<T>(qchunk(g, k, 1), kq[1], dot16<T>(qchunk(g, k, 0), kq[0], dots[g]));
            }
          }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float acc = 0.f;
          if constexpr (kF8) {
            acc = dots[g];
          } else {
#pragma unroll
            for (int k = 0; k < KPL; ++k) acc = dot16<T>(qchunk(g, k, 0), kv[u][k], acc);
          }
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
      for (int k = 0; k < KPL; ++k)
        vv[u][k] = ok[u] ? tile_load(vp + lane + 64 * k) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int bi = b + u;
      if (bi < nb && ok[u]) {
        const int tok0 = (b_begin + bi) * BS + seg * X;  // first token of this lane's segment
        // Tokens past the context in the last block: zero the values so stale
        // cache contents (even NaN bit patterns) cannot leak in.
        if (tok0 + X > L) {
          using E = std::conditional_t<kF8, uint8_t, T>;
#pragma unroll
          for (int k = 0; k < KPL; ++k) {
            union {
              uint4 v;
              E e[X];
            } w;
            w.v = vv[u][k];
#pragma unroll
            for (int e = 0; e < X; ++e)
              if (tok0 + e >= L) w.e[e] = E{};
            vv[u][k] = w.v;
          }
        }
        if constexpr (kF8) {
          // each value row's 16 elements dequantised once for every head,
          // against the segment's 16 probabilities of the head (from LDS)
#pragma unroll
          for (int k = 0; k < KPL; ++k) {
            float vf[16];
            const uint32_t w[4] = {vv[u][k].x, vv[u][k].y, vv[u][k].z, vv[u][k].w};
#pragma unroll
            for (int e = 0; e < 16; ++e) vf[e] = fp8_elem_f32(w[e / 4] >> (8 * (e % 4))) * vs;
            if constexpr (std::is_same_v<T, float>) {
#pragma unroll
              for (int g = 0; g < G; ++g) {
                const float4* pp = reinterpret_cast<const float4*>(&s_p[g][bi * BS + seg * X]);
                float a = acc[g][k];
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                  const float4 t4 = pp[q4];
                  a = fmaf(t4.x, vf[4 * q4], a);
                  a = fmaf(t4.y, vf[4 * q4 + 1], a);
                  a = fmaf(t4.z, vf[4 * q4 + 2], a);
                  a = fmaf(t4.w, vf[4 * q4 + 3], a);
                }
                acc[g][k] = a;
              }
            } else {
              // values and probabilities rounded to the query type, token
              // pairs per v_dot2
              uint4 vq[2];
#pragma unroll
              for (int h = 0; h < 2; ++h)
                vq[h] = make_uint4(pack2_hw<T>(vf[8 * h + 0], vf[8 * h + 1]),
                                   pack2_hw<T>(vf[8 * h + 2], vf[8 * h + 3]),
                                   pack2_hw<T>(vf[8 * h + 4], vf[8 * h + 5]),
                                   pack2_hw<T>(vf[8 * h + 6], vf[8 * h + 7]));
#pragma unroll
              for (int g = 0; g < G; ++g) {
                const float4* pp = reinterpret_cast<const float4*>(&s_p[g][bi * BS + seg * X]);
                float a = acc[g][k];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                  const float4 pa = pp[2 * h], pb = pp[2 * h + 1];
                  const uint4 pk = make_uint4(pack2_hw<T>(pa.x, pa.y), pack2_hw<T>(pa.z, pa.w),
                                              pack2_hw<T>(pb.x, pb.y), pack2_hw<T>(pb.z, pb.w));
                  a = dot16<T>(pk, vq[h], a);
                }
                acc[g][k] = a;
              }
            }
          }
          continue;
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
          } else if constexpr (!kF8) {
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

// ---------------------------------------------------------------------------
// Fast decode path (16-bit caches, and fp8 caches under 16-bit queries,
// whose (block, head) tiles are whole 1 KiB wave loads of at most 8 KiB).
//
// Work list: decode_plan_kernel (one workgroup) turns context_lens into the
// list of (sequence, chunk) items, longest first, a chunk being NW * PT
// tokens, and a small header {0, item count}. All of it lives in the caller's
// workspace and is rebuilt by every call, so the launches can be captured
// in a graph and replayed with new lengths; max_context_len only sizes the
// grid, surplus workgroups exit at once.
//
// paged_decode_rows_kernel: one workgroup of NW waves per (item, kv head);
// the chunk's blocks are split evenly over the waves (up to PT tokens each).
// Per wave, with no cross-lane reduction inside the loops:
//   K pass: stages of 8 16-byte loads per lane, double-buffered; load k of a
//     key tile gives lane l vector l + 64 k, i.e. token l % BS and chunk
//     l / BS + k * (64 / BS), so every instruction reads 1 KiB contiguous and
//     the lane needs only those chunks of q (held in registers). The partial
//     dot products of a token are summed over its 64 / BS lanes with DPP and
//     permlane swaps; logits go to LDS. The first two V stages are issued
//     during the last K stages.
//   softmax: DPP max / sum over the wave's tokens; probabilities are stored
//     in LDS rounded to the cache type.
//   V pass: same 1 KiB-per-instruction loads of the value tiles; lane l owns
//     rows l / (BS/8) + k * 64 / (BS/8) over 8 tokens, and the BS/8 lanes of
//     a row are summed with DPP once at the end.
// The NW partial results are merged in LDS. A sequence of a single chunk
// writes its output directly; a longer one writes one f32 partial row per
// chunk (D values + a 32-float line holding {max (log2 units), sum}, whole
// 128-byte lines), merged by decode_merge_kernel, whose waves read each
// (sequence, head)'s length and skip the single-chunk ones (a list of the
// multi-chunk sequences would put one more dependent load in front of the
// partial rows of this latency-bound launch). (Merging in the last workgroup to finish would need an
// agent-scope release per chunk, which on gfx950 writes back the XCD's L2:
// measured with only that fence added, c3 decode went from 176 to 823 us
// per layer, against 4.7 us for the extra launch.)
// ---------------------------------------------------------------------------
// Floats per split-K partial row of the rows path: D outputs + a 32-float
// line holding {max, sum}.
template <int D>
constexpr int kPartRow = D + 32;

__device__ __forceinline__ int clamp_context(uint32_t ctx, int max_ctx, int cap) {
  return min((int)min(ctx, (uint32_t)max_ctx), cap);
}

// Items are emitted longest first: a counting sort over kPlanBuckets
// classes of chunk length, stable within a class, so full chunks start
// first and the last workgroups the dispatcher hands out are short, which
// keeps the launch's tail short (measured on c3: 8 classes beat 2, 4 and
// 16, and sequence order).
constexpr int kPlanBuckets = 8;

__device__ __forceinline__ int plan_bucket(int L, int p, int part_tokens) {
  if (L <= 0) return kPlanBuckets - 1;
  const int n = min(part_tokens, L - p * part_tokens);  // tokens of chunk p, >= 1
  return (int)(((int64_t)(part_tokens - n) * kPlanBuckets) / part_tokens);
}

__global__ __launch_bounds__(1024) void decode_plan_kernel(
    const uint32_t* __restrict__ context_lens, int32_t num_seqs, int32_t max_ctx,
    int32_t cap_tokens, int32_t part_tokens, uint2* __restrict__ items,
    uint32_t* __restrict__ queue) {
  constexpr int NB = kPlanBuckets;
  __shared__ uint32_t s_wave[16][NB];
  __shared__ uint32_t s_base[NB + 1];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int per = (num_seqs + 1023) / 1024;
  const int s0 = min(tid * per, num_seqs);
  const int s1 = min(s0 + per, num_seqs);
  uint32_t cnt[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) cnt[b] = 0;
  for (int s = s0; s < s1; ++s) {
    const int L = clamp_context(context_lens[s], max_ctx, cap_tokens);
    const int n = L > 0 ? (L + part_tokens - 1) / part_tokens : 1;
    for (int p = 0; p < n; ++p) {
      const int b = plan_bucket(L, p, part_tokens);
#pragma unroll
      for (int c = 0; c < NB; ++c) cnt[c] += c == b;
    }
  }
  // per bucket: exclusive prefix over the threads (wave scan, then waves)
  uint32_t pre[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    uint32_t x = cnt[b];
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t y = __shfl_up(x, off, 64);
      if (lane >= off) x += y;
    }
    pre[b] = x - cnt[b];
    if (lane == 63) s_wave[wave][b] = x;
  }
  __syncthreads();
  if (tid == 0) {
    uint32_t acc = 0;
    for (int b = 0; b < NB; ++b) {
      s_base[b] = acc;
      for (int w = 0; w < 16; ++w) {
        const uint32_t t = s_wave[w][b];
        s_wave[w][b] = acc;
        acc += t;
      }
    }
    s_base[NB] = acc;
  }
  __syncthreads();
  uint32_t pos[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) pos[b] = s_wave[wave][b] + pre[b];
  for (int s = s0; s < s1; ++s) {
    const int L = clamp_context(context_lens[s], max_ctx, cap_tokens);
    const int n = L > 0 ? (L + part_tokens - 1) / part_tokens : 1;
    for (int p = 0; p < n; ++p) {
      const int b = plan_bucket(L, p, part_tokens);
      uint32_t at = 0;
#pragma unroll
      for (int c = 0; c < NB; ++c)
        if (c == b) at = pos[c]++;
      items[at] = make_uint2(((uint32_t)s << 16) | (uint32_t)p, (uint32_t)max(L, 0));
    }
  }
  if (tid == 0) {
    queue[0] = 0u;
    queue[1] = s_base[NB];
  }
}

#ifndef VPA_DECODE_MERGE_WAVES_PER_CU
#define VPA_DECODE_MERGE_WAVES_PER_CU 16
#endif
#ifndef VPA_DECODE_NV
#define VPA_DECODE_NV 8
#endif
#ifndef VPA_DECODE_FP8_NV
#define VPA_DECODE_FP8_NV 4
#endif
#ifndef VPA_DECODE_ROWS_WAVES_PER_EU
#define VPA_DECODE_ROWS_WAVES_PER_EU 3
#endif

// Workgroup of NW waves = one (sequence, kv head, chunk of NW * PT tokens)
// work unit. Wave w attends over partition w of the chunk (PT tokens); the NW
// partial results are merged in LDS, so HBM partial rows are only written for
// sequences longer than one chunk.
//
// C is the cache element type: T itself, or fp8_t (E4M3FN bytes, 16 per
// vector). With fp8 each 16-byte K or V vector is converted once to two
// vectors of T (exact, v_cvt_scalef32_pk_*_fp8 with scale 1) and the same
// v_dot2 products follow; a lane's q chunk is then 16 dims (two vectors),
// *k_scale is folded into the softmax scale and *v_scale into the output.
// Waves per SIMD the rows kernel is compiled for: instances with many q
// vectors per lane (16-byte vectors: G x chunks per lane, two per chunk for
// fp8) would spill at 3 (with 512-token waves: 16 and more).
#ifndef VPA_DECODE_FP8_WAVES_PER_EU
#define VPA_DECODE_FP8_WAVES_PER_EU VPA_DECODE_ROWS_WAVES_PER_EU
#endif
template <typename C, int D, int BS, int G>
constexpr int rows_waves_per_eu() {
  constexpr bool f8 = sizeof(C) == 1;
  constexpr int qvec = G * (D * BS / ((f8 ? 16 : 8) * 64)) * (f8 ? 2 : 1);
  return qvec >= 16 ? 2 : f8 ? VPA_DECODE_FP8_WAVES_PER_EU : VPA_DECODE_ROWS_WAVES_PER_EU;
}

// kAppend (16-bit caches): the launch also appends each sequence's new K/V
// row (new_key / new_value, one token per sequence) at position L - 1 of its
// context, the slot vASR's decode metadata gives the step's token
// (paged_kv_cache.rs:985-1017), in place of a reshape_and_cache launch before
// it. The wave whose partition ends at the context's last block holds that
// block's K and V tiles in registers anyway: it stages the two new rows in
// LDS at its start, puts the token's values into the tiles before using
// them, and writes back whole 32-byte sectors with non-temporal stores: the
// 16 key units of the token with their neighbours (tokens 2i, 2i + 1 share a
// sector), and the whole value tile (every 32-byte value row holds the
// token). No partially written sector reaches HBM.
template <typename T, typename C, int D, int BS, int G, int PT, int NW, bool kAppend = false>
__global__ __launch_bounds__(64 * NW)
__attribute__((amdgpu_waves_per_eu(rows_waves_per_eu<C, D, BS, G>())))
void paged_decode_rows_kernel(
    T* __restrict__ out, const T* __restrict__ query, const C* __restrict__ key_cache,
    const C* __restrict__ value_cache, const uint32_t* __restrict__ block_tables,
    int32_t block_table_stride, float scale, int32_t num_heads, int32_t num_kv_heads,
    int64_t num_blocks, int64_t block_stride, int64_t head_stride, float* __restrict__ part_out,
    int32_t max_parts, const uint2* __restrict__ items, const uint32_t* __restrict__ queue,
    int32_t num_seqs, int32_t max_ctx, int32_t cap_tokens, const float* __restrict__ k_scale,
    const float* __restrict__ v_scale, const T* __restrict__ new_key,
    const T* __restrict__ new_value, int64_t new_key_stride, int64_t new_value_stride,
    int32_t kv_rep) {
  constexpr bool kF8 = std::is_same_v<C, fp8_t>;
  static_assert(kF8 || std::is_same_v<C, T>, "cache type is the query type or fp8");
  static_assert(!(kAppend && kF8), "the fused append writes 16-bit caches");
  constexpr int X = pack_x<C>();
  static_assert(X == (kF8 ? 16 : 8), "16-bit or fp8 cache elements only");
  constexpr int PB = PT / BS;        // blocks per wave partition
  // fp8 at 8-token blocks: a 16-byte value vector holds two rows (dims 2r
  // and 2r + 1) of the block's 8 tokens; otherwise VPR vectors make a row.
  constexpr bool kPairRows = kF8 && BS == 8;
  constexpr int VPR = kPairRows ? 1 : BS / X;  // 16-byte vectors per value row
  constexpr int NVV = D * BS / X / 64;          // value vectors per lane per block
  constexpr int NACC = kPairRows ? 2 * NVV : NVV;  // value rows per lane
  constexpr int DSTEP = 64 / VPR;    // row stride between a lane's value vectors
  constexpr int NPL = PT / 64;       // partition tokens per lane in the softmax
  // Stages of NV loads per lane: 8 (8 KiB per wave) for 16-bit caches, 4
  // for fp8, whose stages of 8 hold twice the tokens and twice the
  // conversion and dot-product work between loads (measured: 4 loads per
  // stage 3-5 % faster on fp8 c3 than 8). A K stage reads BKS
  // key tiles: load k of a tile gives lane l vector l + 64k, i.e. token
  // l % BS and 16-byte chunk l / BS + k * (64 / BS), so each instruction
  // reads 1 KiB contiguous and the lane needs only those chunks of q
  // (held in registers); the partial dot products of a token are summed
  // over its 64 / BS lanes with DPP / permlane swaps. A V stage reads BKS
  // value tiles the same way (lane l: row l / (BS/8) + k * 64 / (BS/8),
  // tokens (l % (BS/8)) * 8 .. +7).
  constexpr int KPL = D * BS / (X * 64);  // loads per lane per tile (K or V)
  // 16-byte loads per lane per stage: the whole tiles that fit NV0 loads,
  // at least one tile (head dims 96 and 192 give 3 or 6 loads per tile)
  constexpr int NV0 = kF8 ? VPA_DECODE_FP8_NV : VPA_DECODE_NV;
  constexpr int NV = KPL >= NV0 ? KPL : (NV0 / KPL) * KPL;
  constexpr int LPT = 64 / BS;            // lanes per token in a key tile
  constexpr int BKS = NV / KPL;           // tiles per stage
  static_assert(KPL == NVV && KPL >= 1 && KPL <= NV && NV % KPL == 0, "stage shape");
  static_assert(VPR >= 1 && VPR <= 4 && PB <= 64 && PT % 64 == 0 && PT >= D, "shape");

  __shared__ float s_logit[NW][G][PT];
  __shared__ __align__(16) uint16_t s_p[NW][G][PT];
  __shared__ float s_m[NW][G], s_l[NW][G];
  constexpr int NR = D / 8;  // 16-byte vectors of a new 16-bit K (or V) row
  __shared__ __align__(16) uint4 s_new[kAppend ? 2 * NR : 1];

  const int lane = threadIdx.x & 63;
  // Uniform where a stage holds at most two tiles: the partition bounds,
  // block ids and tile addresses derived from the wave index then stay in
  // scalar registers (with more tiles per stage their addresses would not
  // fit them and spill).
  const int wave = BKS <= 2 ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)
                            : (int)(threadIdx.x >> 6);
  const uint32_t w = blockIdx.x;
  const int j = (int)(w % (uint32_t)num_kv_heads);
  const uint32_t want = w / (uint32_t)num_kv_heads;  // index of this workgroup's item
  // the list holds num_seqs * ceil(max_ctx / 128) >= gridDim.x / num_kv_heads
  // entries, so the item is read together with the count (one round trip)
  const uint32_t nitems = queue[1];
  const uint2 item = items[want];
  // (the empty asm keeps the compiler from sinking the item load below the
  // count test)
  asm volatile("" ::"s"(nitems), "s"(item.x), "s"(item.y));
  if (want >= nitems) return;  // surplus workgroup of the grid
  const int s = (int)(item.x >> 16);
  const int chunk = (int)(item.x & 0xffffu);
  // a work list built by an earlier call is only trusted within this call's
  // bounds (sequence index, context cap), so every access stays in range
  if (s >= num_seqs) return;
  const int L = clamp_context(item.y, max_ctx, cap_tokens);
  if (L <= 0) {
    if (chunk == 0)
      for (int i = threadIdx.x; i < G * D; i += 64 * NW)
        store_from_f32<T>(out + ((int64_t)s * num_heads + j * G) * D + i, 0.f);
    return;
  }
  const int nblk = (L + BS - 1) / BS;
  const int nchunks = (nblk + PB * NW - 1) / (PB * NW);
  // an item past the sequence's chunks (a list built for other lengths or
  // another max_context_len) would write a partial row outside (s, h) or
  // race with chunk 0 on the output: skip it
  if (chunk >= nchunks || chunk >= max_parts) return;
  // the chunk's blocks are split evenly over the NW waves (at most PB each),
  // so short sequences keep every wave busy
  const int c_begin = chunk * PB * NW;
  const int c_nb = min(PB * NW, nblk - c_begin);
  const int b_begin = c_begin + (c_nb * wave) / NW;
  const int nb = c_begin + (c_nb * (wave + 1)) / NW - b_begin;  // 0: idle wave
  // fused append: this wave's partition ends at the context's last block,
  // which holds the new token at offset app_off (a context clamped by
  // max_context_len or the table appends nothing)
  const bool app = kAppend && nb > 0 && b_begin + nb == nblk && item.y == (uint32_t)L;
  const int app_off = (L - 1) % BS;

  float acc[G][NACC];
  float m[G], lsum[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    lsum[g] = 0.f;
#pragma unroll
    for (int k = 0; k < NACC; ++k) acc[g][k] = 0.f;
  }

  float vs = 1.f;  // value scale of an fp8 cache
  if constexpr (kF8) {
    scale *= *k_scale;
    vs = *v_scale;
  }
  // logits are kept in log2 units (scale * log2 e folded in), so every
  // exponential below is one v_exp_f32; the partial rows' maxima are in the
  // same units for decode_merge_kernel
  scale *= 1.4426950408889634f;

  if (nb > 0) {
    // block ids of the partition (lane b holds block b) and this lane's q chunks
    const uint32_t my_bt =
        lane < nb ? block_tables[(int64_t)s * block_table_stride + b_begin + lane] : 0u;
    constexpr int QV = kF8 ? 2 : 1;  // 16-byte vectors of q per chunk
    uint4 qv[G][KPL][QV];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const T* qrow = query + ((int64_t)s * num_heads + j * G + g) * D;
#pragma unroll
      for (int k = 0; k < KPL; ++k)
#pragma unroll
        for (int h2 = 0; h2 < QV; ++h2)
          qv[g][k][h2] =
              *reinterpret_cast<const uint4*>(qrow + (lane / BS + k * LPT) * X + 8 * h2);
    }

    // the new K and V rows of head j (the appending wave's lanes 0 .. 2 NR - 1),
    // loaded before the first tiles so that the wait for those covers them
    uint4 nrow = make_uint4(0u, 0u, 0u, 0u);
    if (kAppend && app && lane < 2 * NR)
      nrow = *reinterpret_cast<const uint4*>(
          lane < NR ? new_key + (int64_t)s * new_key_stride + (int64_t)j * D + lane * 8
                    : new_value + (int64_t)s * new_value_stride + (int64_t)j * D +
                          (lane - NR) * 8);

    // j counts kv_rep replicas of every kv head (more query heads per kv
    // head than G): its cache head is j / kv_rep
    const int64_t head_off = (int64_t)(j / kv_rep) * head_stride;
    const uint4* kbase = reinterpret_cast<const uint4*>(key_cache + head_off);
    const uint4* vbase = reinterpret_cast<const uint4*>(value_cache + head_off);
    const int64_t bstride_v = block_stride / X;
    const int t = lane % BS;     // K: token of this lane within a tile
    const int seg = lane % VPR;  // V: 8-token segment of this lane
    const int nks = (((nb + BKS - 1) / BKS) + 1) & ~1;  // stages per pass, rounded up to even
    float* const my_logit = &s_logit[wave][0][0];
    uint16_t* const my_p = &s_p[wave][0][0];

    // Block id of tile u of stage st (uniform); blocks past the partition
    // or out of the pool read block 0 (in bounds) and are masked when
    // consumed, so loads never branch.
    // (the pool check compares 32 bits, in scalar registers, unless the
    // pool holds more than 2^32 blocks)
    const bool huge_pool = num_blocks > (int64_t)0xffffffffu;
    auto tile_block = [&](int st, int u, bool& ok) -> uint32_t {
      const int bi = st * BKS + u;
      const uint32_t phys = (uint32_t)__builtin_amdgcn_readlane((int)my_bt, bi < nb ? bi : 0);
      ok = bi < nb && (huge_pool || phys < (uint32_t)num_blocks);
      return ok ? phys : 0u;
    };
    auto load_stage = [&](const uint4* base, int st, uint4(&buf)[NV]) {
#pragma unroll
      for (int u = 0; u < BKS; ++u) {
        bool ok;
        const uint4* tp = base + (int64_t)tile_block(st, u, ok) * bstride_v + lane;
#pragma unroll
        for (int k = 0; k < KPL; ++k) buf[u * KPL + k] = tile_load(tp + 64 * k);
      }
    };
    // logits of BKS tiles
    auto compute_k = [&](int st, const uint4(&buf)[NV]) {
#pragma unroll
      for (int u = 0; u < BKS; ++u) {
        bool ok;
        const uint32_t phys = tile_block(st, u, ok);
        const int bi = st * BKS + u;
        const bool valid = ok && (b_begin + bi) * BS + t < L;
        uint4 kt[KPL];
#pragma unroll
        for (int k = 0; k < KPL; ++k) kt[k] = buf[u * KPL + k];
        if constexpr (kAppend) {
          if (app && ok && bi == nb - 1) {  // (uniform) the new token's block
            // lane l holds chunk l / BS + k LPT of token t: the token's
            // lanes take the new row's chunks, then the lanes of its 32-byte
            // sectors write them back whole
            if (t == app_off)
#pragma unroll
              for (int k = 0; k < KPL; ++k) kt[k] = s_new[lane / BS + k * LPT];
            if ((t >> 1) == (app_off >> 1)) {
              uint4* dst = const_cast<uint4*>(kbase) + (int64_t)phys * bstride_v + lane;
#pragma unroll
              for (int k = 0; k < KPL; ++k) tile_store(dst + 64 * k, kt[k]);
            }
          }
        }
        float qk[G];
#pragma unroll
        for (int g = 0; g < G; ++g) qk[g] = 0.f;
#pragma unroll
        for (int k = 0; k < KPL; ++k) {
          if constexpr (kF8) {
            uint4 klo, khi;
            fp8x16_to_pk<T>(kt[k], klo, khi);
#pragma unroll
            for (int g = 0; g < G; ++g)
              qk[g] = dot16<T>(qv[g][k][1], khi, dot16<T>(qv[g][k][0], klo, qk[g]));
          } else {
#pragma unroll
            for (int g = 0; g < G; ++g) qk[g] = dot16<T>(qv[g][k][0], kt[k], qk[g]);
          }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float r = sum_lanes_mod<BS>(qk[g]);
          if (lane < BS && bi < PB) my_logit[g * PT + bi * BS + lane] = valid ? r * scale : -INFINITY;
        }
      }
    };
    // P.V over BKS tiles
    auto compute_v = [&](int st, const uint4(&buf)[NV]) {
#pragma unroll
      for (int u = 0; u < BKS; ++u) {
        bool ok;
        const uint32_t phys = tile_block(st, u, ok);
        if (!ok) continue;
        const int bi = st * BKS + u;
        uint4 vv[NVV];
#pragma unroll
        for (int k = 0; k < NVV; ++k) vv[k] = buf[u * KPL + k];
        if constexpr (kAppend) {
          if (app && bi == nb - 1) {  // (uniform) the new token's block
            // lane l holds rows l / VPR + k DSTEP, tokens seg X .. seg X + X - 1:
            // the lanes of the token's segment put in its values, then the
            // whole tile is written back
            if (seg == app_off / X) {
              const uint16_t* nv = reinterpret_cast<const uint16_t*>(&s_new[NR]);
#pragma unroll
              for (int k = 0; k < NVV; ++k)
                vv[k] = put_u16(vv[k], app_off % X, nv[lane / VPR + k * DSTEP]);
            }
            uint4* dst = const_cast<uint4*>(vbase) + (int64_t)phys * bstride_v + lane;
#pragma unroll
            for (int k = 0; k < NVV; ++k) tile_store(dst + 64 * k, vv[k]);
          }
        }
        if constexpr (kPairRows) {
          // vector k of lane l: rows 2 (l + 64 k) and 2 (l + 64 k) + 1, the
          // block's 8 tokens each, against the block's 8 probabilities
          const int tok0 = (b_begin + bi) * BS;
#pragma unroll
          for (int k = 0; k < NVV; ++k) {
            uint4 vh[2];
            fp8x16_to_pk<T>(vv[k], vh[0], vh[1]);
            if (tok0 + BS > L) {  // past the context in the last block: stale values
#pragma unroll
              for (int h2 = 0; h2 < 2; ++h2) {
                union {
                  uint4 v;
                  uint16_t e[8];
                } wv;
                wv.v = vh[h2];
#pragma unroll
                for (int e = 0; e < 8; ++e)
                  if (tok0 + e >= L) wv.e[e] = 0;
                vh[h2] = wv.v;
              }
            }
#pragma unroll
            for (int g = 0; g < G; ++g) {
              const uint4 pk = *reinterpret_cast<const uint4*>(&my_p[g * PT + bi * BS]);
              acc[g][2 * k] = dot16<T>(pk, vh[0], acc[g][2 * k]);
              acc[g][2 * k + 1] = dot16<T>(pk, vh[1], acc[g][2 * k + 1]);
            }
          }
          continue;
        }
        const int tok0 = (b_begin + bi) * BS + seg * X;
        if constexpr (kF8) {
#pragma unroll
          for (int k = 0; k < NVV; ++k) {
            uint4 vh[2];
            fp8x16_to_pk<T>(vv[k], vh[0], vh[1]);
            if (tok0 + X > L) {  // past the context in the last block: stale values
#pragma unroll
              for (int h2 = 0; h2 < 2; ++h2) {
                union {
                  uint4 v;
                  uint16_t e[8];
                } wv;
                wv.v = vh[h2];
#pragma unroll
                for (int e = 0; e < 8; ++e)
                  if (tok0 + 8 * h2 + e >= L) wv.e[e] = 0;
                vh[h2] = wv.v;
              }
            }
#pragma unroll
            for (int g = 0; g < G; ++g) {
              const uint4* pp = reinterpret_cast<const uint4*>(&my_p[g * PT + bi * BS + seg * X]);
              acc[g][k] = dot16<T>(pp[1], vh[1], dot16<T>(pp[0], vh[0], acc[g][k]));
            }
          }
          continue;
        }
        if (tok0 + X > L) {
          // past the context in the last block: zero the values (stale contents)
#pragma unroll
          for (int k = 0; k < NVV; ++k) {
            union {
              uint4 v;
              uint16_t e[8];
            } wv;
            wv.v = vv[k];
#pragma unroll
            for (int e = 0; e < X; ++e)
              if (tok0 + e >= L) wv.e[e] = 0;
            vv[k] = wv.v;
          }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const uint4 pk = *reinterpret_cast<const uint4*>(&my_p[g * PT + bi * BS + seg * X]);
#pragma unroll
          for (int k = 0; k < NVV; ++k) acc[g][k] = dot16<T>(pk, vv[k], acc[g][k]);
        }
      }
    };

    // ---- software pipeline (nks even): the next stage's loads are in
    // flight while the current stage is computed; the first two V stages are
    // issued during the last two K stages, before the softmax ----
    uint4 bufA[NV], bufB[NV];
    load_stage(kbase, 0, bufA);
    load_stage(kbase, 1, bufB);
    if (kAppend && app) {
      if (lane < 2 * NR) s_new[lane] = nrow;
      lds_wave_sync();
    }
    for (int st = 0; st + 2 < nks; st += 2) {
      compute_k(st, bufA);
      load_stage(kbase, st + 2, bufA);
      compute_k(st + 1, bufB);
      load_stage(kbase, st + 3, bufB);
    }
    compute_k(nks - 2, bufA);
    load_stage(vbase, 0, bufA);
    compute_k(nks - 1, bufB);
    load_stage(vbase, 1, bufB);

    // ---- softmax over the partition ----
    lds_wave_sync();
    {
      const int ntok = nb * BS;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float v[NPL];
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < NPL; ++i) {
          const int idx = i * 64 + lane;
          v[i] = idx < ntok ? my_logit[g * PT + idx] : -INFINITY;
          mx = fmaxf(mx, v[i]);
        }
        mx = wave_max_dpp(mx);
        float sm = 0.f;
#pragma unroll
        for (int i = 0; i < NPL; ++i) {
          if (i * 64 >= ntok) break;  // (uniform) the P.V pass reads only the first ntok
          const float p = v[i] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(v[i] - mx);
          sm += p;
          T pt;
          store_from_f32<T>(&pt, p);
          my_p[g * PT + i * 64 + lane] = pt.x;
        }
        m[g] = mx;
        lsum[g] = wave_sum_dpp(sm);
      }
    }
    lds_wave_sync();

    for (int st = 0; st + 2 < nks; st += 2) {
      compute_v(st, bufA);
      load_stage(vbase, st + 2, bufA);
      compute_v(st + 1, bufB);
      load_stage(vbase, st + 3, bufB);
    }
    compute_v(nks - 2, bufA);
    compute_v(nks - 1, bufB);

    // sum the VPR lanes that hold the same value row
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int k = 0; k < NACC; ++k) {
        if constexpr (VPR >= 2) acc[g][k] += dpp<kDppQuadXor1>(acc[g][k]);
        if constexpr (VPR >= 4) acc[g][k] += dpp<kDppQuadXor2>(acc[g][k]);
        if constexpr (kF8) acc[g][k] *= vs;
      }
  }

  // ---- merge the NW partitions of the chunk in LDS ----
  // Each wave leaves its unnormalised output (in its own s_logit slot, free
  // after the softmax) and its max / sum; then the workgroup combines them.
  // The barriers wait for LDS only: __syncthreads() would also wait for this
  // wave's outstanding global stores (the fused append's sector writes),
  // which nothing here reads.
  lds_barrier();
  {
    float* my_row = &s_logit[wave][0][0];
    if constexpr (kPairRows) {
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int k = 0; k < NACC; ++k) my_row[g * D + 2 * (lane + 64 * (k / 2)) + k % 2] = acc[g][k];
    } else {
      const int row0 = lane / VPR;
      if (lane % VPR == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int k = 0; k < NVV; ++k) my_row[g * D + row0 + k * DSTEP] = acc[g][k];
      }
    }
    if (lane == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        s_m[wave][g] = m[g];
        s_l[wave][g] = lsum[g];
      }
    }
  }
  lds_barrier();
  // thread e of the workgroup combines output elements e, e + 64*NW, ...
  // (contiguous per head row, so stores write whole lines)
  const bool single = nchunks == 1;
  for (int e = threadIdx.x; e < G * D; e += 64 * NW) {
    const int g = e / D, d = e - (e / D) * D;
    float mx = -INFINITY;
#pragma unroll
    for (int q = 0; q < NW; ++q) mx = fmaxf(mx, s_m[q][g]);
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int q = 0; q < NW; ++q) {
      const float wq = s_m[q][g] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s_m[q][g] - mx);
      num = fmaf(wq, s_logit[q][0][g * D + d], num);
      den = fmaf(wq, s_l[q][g], den);
    }
    const int h = j * G + g;
    if (single) {
      store_from_f32<T>(out + ((int64_t)s * num_heads + h) * D + d, num / (den + 1e-6f));
    } else {
      // split-K partial row: D floats of unnormalised output, then one
      // 128-byte line {max, sum, 0...} (whole lines: partial-line stores
      // cost a read-modify-write in HBM)
      float* prow = part_out + (((int64_t)s * num_heads + h) * max_parts + chunk) * kPartRow<D>;
      prow[d] = num;
      if (d < 32) prow[D + d] = d == 0 ? mx : (d == 1 ? den : 0.f);
    }
  }
}

// One wave per (query head, sequence) with more than one partition: merge of
// the generic kernel's split-K partials.
template <typename T, int D>
__global__ __launch_bounds__(64) void paged_decode_reduce_kernel(
    T* __restrict__ out, const uint32_t* __restrict__ context_lens, int32_t max_ctx,
    int32_t block_table_stride, int32_t block_size, int32_t num_heads,
    const float* __restrict__ part_out, const float* __restrict__ part_max,
    const float* __restrict__ part_sum, int32_t max_parts, int32_t part_tokens) {
  __shared__ float s_w[kDecodeMaxPartitions];
  const int lane = threadIdx.x;
  const int h = blockIdx.x;
  const int s = blockIdx.y;
  const int L = min((int)min(context_lens[s], (uint32_t)max_ctx), block_table_stride * block_size);
  const int nparts = (L + part_tokens - 1) / part_tokens;
  if (nparts <= 1) return;

  const int64_t row0 = ((int64_t)s * num_heads + h) * max_parts;
  float mx = -INFINITY;
  for (int p = lane; p < nparts; p += 64) mx = fmaxf(mx, part_max[row0 + p]);
  mx = wave_max_dpp(mx);
  float tot = 0.f;
  for (int p = lane; p < nparts; p += 64) {
    const float pm = part_max[row0 + p];
    const float w = pm == -INFINITY ? 0.f : expf(pm - mx);
    s_w[p] = w;
    tot += w * part_sum[row0 + p];
  }
  tot = wave_sum_dpp(tot);
  lds_wave_sync();
  const float inv = 1.f / (tot + 1e-6f);
  T* orow = out + ((int64_t)s * num_heads + h) * D;
  for (int d = lane; d < D; d += 64) {
    float a = 0.f;
    for (int p = 0; p < nparts; ++p) a = fmaf(s_w[p], part_out[(row0 + p) * D + d], a);
    store_from_f32<T>(orow + d, a * inv);
  }
}

// 16-bit caches: 4 waves of up to 512 tokens per 2048-token chunk (measured
// on c3 with the longest-first plan: 172.5 us per layer; 8 x 512 174.2,
// 4 x 448 173.0, 4 x 384 174.0, 4 x 256 174.7, 6 x 512 179.7; 8 x 128 in
// sequence order 175.5)
#ifndef VPA_DECODE_ROWS_PT
#define VPA_DECODE_ROWS_PT 512
#endif
#ifndef VPA_DECODE_ROWS_WAVES
#define VPA_DECODE_ROWS_WAVES 4
#endif
constexpr int kRowsPT = VPA_DECODE_ROWS_PT;  // partition tokens per wave of the rows kernel
constexpr int kRowsWaves = VPA_DECODE_ROWS_WAVES;  // waves (partitions) per workgroup
// fp8 caches: the same chunk, so one work list serves every cache type
// (measured on c3, us per layer: 4 x 512 101.7, 2 x 1024 103.6, 2 x 768 105.8,
// 1 x 1024 107.1; 2 x 512 over 1024-token chunks 102.6)
#ifndef VPA_DECODE_FP8_WAVES
#define VPA_DECODE_FP8_WAVES 4
#endif
#ifndef VPA_DECODE_FP8_PT
#define VPA_DECODE_FP8_PT 512
#endif
constexpr int kF8Waves = VPA_DECODE_FP8_WAVES;
constexpr int kF8PT = VPA_DECODE_FP8_PT;
static_assert(kRowsPT >= kDecodeMinPartitionTokens && kF8PT >= kDecodeMinPartitionTokens,
              "workspace sized for 128-token partitions");
// Tokens per work item (workgroup) of the plan.
constexpr int kDecodeChunk = kRowsPT * kRowsWaves;
static_assert(kF8PT * kF8Waves == kDecodeChunk, "one work list serves every cache type");

// Merge of split-K partials: persistent waves over (sequence, query head)
// units; sequences of one chunk were written directly and are skipped. One
// pass with an online max: each step loads the stats and the rows of up to
// kMergeRows partials together, so a unit costs two dependent loads
// (the context length, then its partials) before the store.
constexpr int kMergeRows = 8;

template <typename T, int D>
__global__ __launch_bounds__(64) void decode_merge_kernel(
    T* __restrict__ out, const uint32_t* __restrict__ context_lens, int32_t num_seqs,
    int32_t max_ctx, int32_t cap_tokens, int32_t part_tokens, int32_t num_heads,
    const float* __restrict__ part, int32_t max_parts) {
  constexpr int DPL = (D + 63) / 64;  // output elements per lane (the last partly, at D 96)
  constexpr int RS = kPartRow<D>;
  constexpr int R = kMergeRows;
  const int lane = threadIdx.x;
  const uint32_t units = (uint32_t)num_seqs * (uint32_t)num_heads;
  for (uint32_t u = blockIdx.x; u < units; u += gridDim.x) {
    const int s = (int)(u / (uint32_t)num_heads);
    const int h = (int)(u % (uint32_t)num_heads);
    const int L = clamp_context(context_lens[s], max_ctx, cap_tokens);
    const int nparts = (L + part_tokens - 1) / part_tokens;
    if (nparts <= 1) continue;
    const float* rows = part + ((int64_t)s * num_heads + h) * max_parts * RS;
    float mx = -INFINITY, tot = 0.f;
    float a[DPL];
#pragma unroll
    for (int k = 0; k < DPL; ++k) a[k] = 0.f;
    for (int c0 = 0; c0 < nparts; c0 += R) {
      const int cn = min(R, nparts - c0);
      float pm[R], pl[R], v[R][DPL];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float* row = rows + (int64_t)(c0 + min(r, cn - 1)) * RS;
        pm[r] = r < cn ? row[D] : -INFINITY;
        pl[r] = row[D + 1];
#pragma unroll
        for (int k = 0; k < DPL; ++k) v[r][k] = lane + 64 * k < D ? row[lane + 64 * k] : 0.f;
      }
      float cm = mx;
#pragma unroll
      for (int r = 0; r < R; ++r) cm = fmaxf(cm, pm[r]);
      if (cm == -INFINITY) continue;  // no token in these partials
      const float rescale = mx == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mx - cm);
      tot *= rescale;
#pragma unroll
      for (int k = 0; k < DPL; ++k) a[k] *= rescale;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float wgt = pm[r] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(pm[r] - cm);
        tot = fmaf(wgt, pl[r], tot);
#pragma unroll
        for (int k = 0; k < DPL; ++k) a[k] = fmaf(wgt, v[r][k], a[k]);
      }
      mx = cm;
    }
    const float inv = 1.f / (tot + 1e-6f);
    T* orow = out + ((int64_t)s * num_heads + h) * D + lane;
#pragma unroll
    for (int k = 0; k < DPL; ++k)
      if (lane + 64 * k < D) store_from_f32<T>(orow + 64 * k, a[k] * inv);
  }
}

// Shapes whose rows kernel takes the fused append: at least 2 KiB of 16-bit
// (block, head) tile, i.e. at most two tiles per 8-load stage (more tiles per
// stage spill scalar registers with the append's extra state).
constexpr bool fused_append_shape(int d, int bs) { return d * bs >= 2048; }

template <typename T, typename C, int D, int BS, int G>
hipError_t launch_decode_rows_c(void* out, const void* q, const void* kc, const void* vc,
                                const uint32_t* bt, int32_t bts, const uint32_t* cl,
                                int32_t max_ctx, float scale, int32_t num_seqs,
                                int32_t num_heads, const CacheGeom& g, const DecodeWorkspace& ws,
                                hipStream_t stream, const float* k_scale, const float* v_scale,
                                const DecodeAppend* app) {
  constexpr bool kFp8 = std::is_same_v<C, fp8_t>;
  constexpr int PT = kFp8 ? kF8PT : kRowsPT;
  constexpr int NW = kFp8 ? kF8Waves : kRowsWaves;
  constexpr int kChunk = PT * NW;  // tokens per workgroup
  static_assert(kChunk == kDecodeChunk, "the plan's chunk");
  const int cap_tokens = bts * g.block_size;
  hipError_t e = hipSuccess;
  if (!ws.planned) {
    hipLaunchKernelGGL(decode_plan_kernel, dim3(1), dim3(1024), 0, stream, cl, num_seqs,
                       max_ctx, cap_tokens, kChunk, ws.items, ws.queue);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const int max_chunks = max(1, (max_ctx + kChunk - 1) / kChunk);
  const int64_t units = (int64_t)num_seqs * max_chunks * g.num_kv_heads;
  if constexpr (!kFp8 && fused_append_shape(D, BS)) {
    if (app != nullptr) {
      hipLaunchKernelGGL((paged_decode_rows_kernel<T, C, D, BS, G, PT, NW, true>),
                         dim3((unsigned)units), dim3(64 * NW), 0, stream, static_cast<T*>(out),
                         static_cast<const T*>(q), static_cast<const C*>(kc),
                         static_cast<const C*>(vc), bt, bts, scale, num_heads, g.num_kv_heads,
                         g.num_blocks, g.block_stride, g.head_stride, ws.part_out,
                         ws.max_parts, ws.items, ws.queue, num_seqs, max_ctx, cap_tokens,
                         k_scale, v_scale, static_cast<const T*>(app->key),
                         static_cast<const T*>(app->value), app->key_token_stride,
                         app->value_token_stride, g.kv_rep);
    }
  }
  if (kFp8 || !fused_append_shape(D, BS) || app == nullptr) {
    hipLaunchKernelGGL((paged_decode_rows_kernel<T, C, D, BS, G, PT, NW>),
                       dim3((unsigned)units), dim3(64 * NW), 0, stream, static_cast<T*>(out),
                       static_cast<const T*>(q), static_cast<const C*>(kc),
                       static_cast<const C*>(vc), bt, bts, scale, num_heads, g.num_kv_heads,
                       g.num_blocks, g.block_stride, g.head_stride, ws.part_out, ws.max_parts,
                       ws.items, ws.queue, num_seqs, max_ctx, cap_tokens, k_scale, v_scale,
                       static_cast<const T*>(nullptr), static_cast<const T*>(nullptr),
                       (int64_t)0, (int64_t)0, g.kv_rep);
  }
  e = hipGetLastError();
  if (e != hipSuccess || max_chunks <= 1) return e;
  const int64_t munits = (int64_t)num_seqs * num_heads;
  const int64_t mwaves =
      std::min<int64_t>(munits, (int64_t)device_cu_count() * VPA_DECODE_MERGE_WAVES_PER_CU);
  hipLaunchKernelGGL((decode_merge_kernel<T, D>), dim3((unsigned)mwaves), dim3(64), 0, stream,
                     static_cast<T*>(out), cl, num_seqs, max_ctx, cap_tokens, kChunk, num_heads,
                     ws.part_out, ws.max_parts);
  return hipGetLastError();
}

template <typename T, int D, int BS, int G>
hipError_t launch_decode_rows(void* out, const void* q, const void* kc, const void* vc,
                              const uint32_t* bt, int32_t bts, const uint32_t* cl,
                              int32_t max_ctx, float scale, int32_t num_seqs, int32_t num_heads,
                              const CacheGeom& g, const DecodeWorkspace& ws, hipStream_t stream,
                              const float* k_scale, const float* v_scale,
                              const DecodeAppend* app) {
  return launch_decode_rows_c<T, T, D, BS, G>(out, q, kc, vc, bt, bts, cl, max_ctx, scale,
                                              num_seqs, num_heads, g, ws, stream, k_scale,
                                              v_scale, app);
}
template <typename T, int D, int BS, int G>
hipError_t launch_decode_rows_fp8(void* out, const void* q, const void* kc, const void* vc,
                                  const uint32_t* bt, int32_t bts, const uint32_t* cl,
                                  int32_t max_ctx, float scale, int32_t num_seqs,
                                  int32_t num_heads, const CacheGeom& g,
                                  const DecodeWorkspace& ws, hipStream_t stream,
                                  const float* k_scale, const float* v_scale,
                                  const DecodeAppend*) {
  return launch_decode_rows_c<T, fp8_t, D, BS, G>(out, q, kc, vc, bt, bts, cl, max_ctx, scale,
                                                  num_seqs, num_heads, g, ws, stream, k_scale,
                                                  v_scale, nullptr);
}

template <typename T, typename C, int D, int BS, int G>
hipError_t launch_decode_tc(void* out, const void* q, const void* kc, const void* vc,
                            const uint32_t* bt, int32_t bts, const uint32_t* cl, int32_t max_ctx,
                            float scale, int32_t num_seqs, int32_t num_heads, const CacheGeom& g,
                            const DecodeWorkspace& ws, hipStream_t stream, const float* k_scale,
                            const float* v_scale, const DecodeAppend*) {
  const int max_parts = (max_ctx + kPT - 1) / kPT;
  dim3 grid((unsigned)g.num_kv_heads, (unsigned)num_seqs, (unsigned)(max_parts > 0 ? max_parts : 1));
  hipLaunchKernelGGL((paged_decode_kernel<T, C, D, BS, G>), grid, dim3(64), 0, stream,
                     static_cast<T*>(out), static_cast<const T*>(q), static_cast<const C*>(kc),
                     static_cast<const C*>(vc), bt, bts, cl, max_ctx, scale, num_heads,
                     g.num_blocks, g.block_stride, g.head_stride, ws.part_out, ws.part_max,
                     ws.part_sum, ws.max_parts, g.kv_rep, k_scale, v_scale);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || max_parts <= 1) return e;
  dim3 rgrid((unsigned)num_heads, (unsigned)num_seqs);
  hipLaunchKernelGGL((paged_decode_reduce_kernel<T, D>), rgrid, dim3(64), 0, stream,
                     static_cast<T*>(out), cl, max_ctx, bts, g.block_size, num_heads, ws.part_out,
                     ws.part_max, ws.part_sum, ws.max_parts, kPT);
  return hipGetLastError();
}

template <typename T, int D, int BS, int G>
hipError_t launch_decode_t(void* out, const void* q, const void* kc, const void* vc,
                           const uint32_t* bt, int32_t bts, const uint32_t* cl, int32_t max_ctx,
                           float scale, int32_t num_seqs, int32_t num_heads, const CacheGeom& g,
                           const DecodeWorkspace& ws, hipStream_t stream, const float* k_scale,
                           const float* v_scale, const DecodeAppend* app) {
  return launch_decode_tc<T, T, D, BS, G>(out, q, kc, vc, bt, bts, cl, max_ctx, scale, num_seqs,
                                          num_heads, g, ws, stream, k_scale, v_scale, app);
}
template <int D, int BS, int G>
hipError_t launch_decode_f32_fp8(void* out, const void* q, const void* kc, const void* vc,
                                 const uint32_t* bt, int32_t bts, const uint32_t* cl,
                                 int32_t max_ctx, float scale, int32_t num_seqs,
                                 int32_t num_heads, const CacheGeom& g, const DecodeWorkspace& ws,
                                 hipStream_t stream, const float* k_scale, const float* v_scale,
                                 const DecodeAppend* app) {
  return launch_decode_tc<float, fp8_t, D, BS, G>(out, q, kc, vc, bt, bts, cl, max_ctx, scale,
                                                  num_seqs, num_heads, g, ws, stream, k_scale,
                                                  v_scale, app);
}

template <typename T, int D, int BS, int G>
hipError_t launch_decode_generic_fp8(void* out, const void* q, const void* kc, const void* vc,
                                     const uint32_t* bt, int32_t bts, const uint32_t* cl,
                                     int32_t max_ctx, float scale, int32_t num_seqs,
                                     int32_t num_heads, const CacheGeom& g,
                                     const DecodeWorkspace& ws, hipStream_t stream,
                                     const float* k_scale, const float* v_scale,
                                     const DecodeAppend* app) {
  return launch_decode_tc<T, fp8_t, D, BS, G>(out, q, kc, vc, bt, bts, cl, max_ctx, scale,
                                              num_seqs, num_heads, g, ws, stream, k_scale,
                                              v_scale, app);
}

#define VPA_DECODE_G(T, D, BS)                                          \
  if (group == 1) return launch_decode_t<T, D, BS, 1>(args...);         \
  if (group == 2) return launch_decode_t<T, D, BS, 2>(args...);         \
  if (group == 4) return launch_decode_t<T, D, BS, 4>(args...);

#define VPA_DECODE_ROWS_G(T, D, BS)                                  \
  if (group == 1) return launch_decode_rows<T, D, BS, 1>(args...);   \
  if (group == 2) return launch_decode_rows<T, D, BS, 2>(args...);   \
  if (group == 4) return launch_decode_rows<T, D, BS, 4>(args...);

// 16-bit caches use the rows kernel wherever a (block, head) tile is at
// most 8 KiB, i.e. 8 wave loads per lane (rows_kernel_shape); f32 and the
// two larger 16-bit tiles (head dims 192 and 256 at 32-token blocks) the
// generic kernel. (Head dim 96 at 16-bit needs blocks of 16 or 32 tokens: a
// tile is a whole number of 1 KiB wave loads.)
#define VPA_DECODE_DBS16(T)                                   \
  if (D == 64 && BS == 8) { VPA_DECODE_ROWS_G(T, 64, 8) }     \
  if (D == 64 && BS == 16) { VPA_DECODE_ROWS_G(T, 64, 16) }   \
  if (D == 64 && BS == 32) { VPA_DECODE_ROWS_G(T, 64, 32) }   \
  if (D == 128 && BS == 8) { VPA_DECODE_ROWS_G(T, 128, 8) }   \
  if (D == 128 && BS == 16) { VPA_DECODE_ROWS_G(T, 128, 16) } \
  if (D == 128 && BS == 32) { VPA_DECODE_ROWS_G(T, 128, 32) } \
  if (D == 96 && BS == 16) { VPA_DECODE_ROWS_G(T, 96, 16) }   \
  if (D == 96 && BS == 32) { VPA_DECODE_ROWS_G(T, 96, 32) }   \
  if (D == 192 && BS == 8) { VPA_DECODE_ROWS_G(T, 192, 8) }   \
  if (D == 192 && BS == 16) { VPA_DECODE_ROWS_G(T, 192, 16) } \
  if (D == 192 && BS == 32) { VPA_DECODE_G(T, 192, 32) }      \
  if (D == 256 && BS == 8) { VPA_DECODE_ROWS_G(T, 256, 8) }   \
  if (D == 256 && BS == 16) { VPA_DECODE_ROWS_G(T, 256, 16) } \
  if (D == 256 && BS == 32) { VPA_DECODE_G(T, 256, 32) }

#define VPA_DECODE_DBS(T)                                   \
  if (D == 64 && BS == 8) { VPA_DECODE_G(T, 64, 8) }        \
  if (D == 64 && BS == 16) { VPA_DECODE_G(T, 64, 16) }      \
  if (D == 64 && BS == 32) { VPA_DECODE_G(T, 64, 32) }      \
  if (D == 128 && BS == 8) { VPA_DECODE_G(T, 128, 8) }      \
  if (D == 128 && BS == 16) { VPA_DECODE_G(T, 128, 16) }    \
  if (D == 128 && BS == 32) { VPA_DECODE_G(T, 128, 32) }    \
  if (D == 96 && BS == 8) { VPA_DECODE_G(T, 96, 8) }        \
  if (D == 96 && BS == 16) { VPA_DECODE_G(T, 96, 16) }      \
  if (D == 96 && BS == 32) { VPA_DECODE_G(T, 96, 32) }      \
  if (D == 192 && BS == 8) { VPA_DECODE_G(T, 192, 8) }      \
  if (D == 192 && BS == 16) { VPA_DECODE_G(T, 192, 16) }    \
  if (D == 192 && BS == 32) { VPA_DECODE_G(T, 192, 32) }    \
  if (D == 256 && BS == 8) { VPA_DECODE_G(T, 256, 8) }      \
  if (D == 256 && BS == 16) { VPA_DECODE_G(T, 256, 16) }    \
  if (D == 256 && BS == 32) { VPA_DECODE_G(T, 256, 32) }

#define VPA_DECODE_FP8_G(T, D, BS)                                       \
  if (group == 1) return launch_decode_rows_fp8<T, D, BS, 1>(args...);   \
  if (group == 2) return launch_decode_rows_fp8<T, D, BS, 2>(args...);   \
  if (group == 4) return launch_decode_rows_fp8<T, D, BS, 4>(args...);

#define VPA_DECODE_GENERIC_FP8_G(T, D, BS)                                    \
  if (group == 1) return launch_decode_generic_fp8<T, D, BS, 1>(args...);     \
  if (group == 2) return launch_decode_generic_fp8<T, D, BS, 2>(args...);     \
  if (group == 4) return launch_decode_generic_fp8<T, D, BS, 4>(args...);

// fp8 shapes (decode_fp8_shape): a whole number of 1 KiB wave loads per
// (block, head) tile, on the rows kernel where the 16-bit decode of the
// shape uses it too (the work list is the same for every cache type), on
// the generic kernel where it does not (head dims 192 and 256 at 32-token
// blocks).
#define VPA_DECODE_FP8_DBS(T)                                  \
  if (D == 64 && BS == 16) { VPA_DECODE_FP8_G(T, 64, 16) }     \
  if (D == 64 && BS == 32) { VPA_DECODE_FP8_G(T, 64, 32) }     \
  if (D == 128 && BS == 16) { VPA_DECODE_FP8_G(T, 128, 16) }   \
  if (D == 128 && BS == 32) { VPA_DECODE_FP8_G(T, 128, 32) }   \
  if (D == 128 && BS == 8) { VPA_DECODE_FP8_G(T, 128, 8) }     \
  if (D == 96 && BS == 32) { VPA_DECODE_FP8_G(T, 96, 32) }     \
  if (D == 192 && BS == 16) { VPA_DECODE_FP8_G(T, 192, 16) }   \
  if (D == 256 && BS == 8) { VPA_DECODE_FP8_G(T, 256, 8) }     \
  if (D == 256 && BS == 16) { VPA_DECODE_FP8_G(T, 256, 16) }   \
  if (D == 192 && BS == 32) { VPA_DECODE_GENERIC_FP8_G(T, 192, 32) } \
  if (D == 256 && BS == 32) { VPA_DECODE_GENERIC_FP8_G(T, 256, 32) }

#define VPA_DECODE_F32_FP8_G(D, BS)                                       \
  if (group == 1) return launch_decode_f32_fp8<D, BS, 1>(args...);        \
  if (group == 2) return launch_decode_f32_fp8<D, BS, 2>(args...);        \
  if (group == 4) return launch_decode_f32_fp8<D, BS, 4>(args...);

// fp8 caches: the rows kernel for bf16 / f16 queries (the generic split-K
// kernel at head dims 192 and 256 with 32-token blocks); f32 queries on the
// generic kernel (decode_f32_fp8_shape).
template <typename... A>
hipError_t dispatch_decode_fp8(int dtype, int D, int BS, int group, A... args) {
  if (dtype == VPA_DTYPE_BF16) { VPA_DECODE_FP8_DBS(bf16_t) }
  if (dtype == VPA_DTYPE_F16) { VPA_DECODE_FP8_DBS(f16_t) }
  if (dtype == VPA_DTYPE_F32) {
    if (D == 64 && BS == 16) { VPA_DECODE_F32_FP8_G(64, 16) }
    if (D == 64 && BS == 32) { VPA_DECODE_F32_FP8_G(64, 32) }
    if (D == 96 && BS == 32) { VPA_DECODE_F32_FP8_G(96, 32) }
    if (D == 128 && BS == 16) { VPA_DECODE_F32_FP8_G(128, 16) }
    if (D == 128 && BS == 32) { VPA_DECODE_F32_FP8_G(128, 32) }
    if (D == 192 && BS == 16) { VPA_DECODE_F32_FP8_G(192, 16) }
    if (D == 192 && BS == 32) { VPA_DECODE_F32_FP8_G(192, 32) }
    if (D == 256 && BS == 16) { VPA_DECODE_F32_FP8_G(256, 16) }
  }
  return hipErrorInvalidValue;
}

template <typename... A>
hipError_t dispatch_decode(int dtype, int D, int BS, int group, A... args) {
  if (dtype == VPA_DTYPE_BF16) { VPA_DECODE_DBS16(bf16_t) }
  if (dtype == VPA_DTYPE_F16) { VPA_DECODE_DBS16(f16_t) }
  if (dtype == VPA_DTYPE_F32) { VPA_DECODE_DBS(float) }
  return hipErrorInvalidValue;
}

#ifndef VPA_READ_NV
#define VPA_READ_NV 8
#endif
// Read ceiling of the decode's access pattern: the rows kernel's work items
// and split of a chunk's blocks over its waves, each wave reading every K
// then every V tile of its blocks with the same 16-byte loads (KPL per lane
// per tile, each instruction 1 KiB contiguous), stages of NV loads double
// buffered, and nothing computed but an XOR of the bytes. The checksum is
// stored only when it equals `magic`, so the loads cannot be dropped.
template <int BS, int KPL>
__global__ __launch_bounds__(64 * kRowsWaves) void paged_read_kernel(
    const uint4* __restrict__ key_cache, const uint4* __restrict__ value_cache,
    const uint32_t* __restrict__ block_tables, int32_t block_table_stride,
    int32_t num_kv_heads, int64_t num_blocks, int64_t block_stride_v, int64_t head_stride_v,
    const uint2* __restrict__ items, const uint32_t* __restrict__ queue, int32_t num_seqs,
    int32_t max_ctx, int32_t cap_tokens, uint32_t magic, uint32_t* __restrict__ sink) {
  constexpr int NW = kRowsWaves;
  constexpr int PB = kRowsPT / BS;  // blocks per wave partition
  constexpr int NV = VPA_READ_NV;    // loads per lane per stage
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const uint32_t w = blockIdx.x;
  const int j = (int)(w % (uint32_t)num_kv_heads);
  const uint32_t want = w / (uint32_t)num_kv_heads;
  const uint32_t nitems = queue[1];
  const uint2 item = items[want];
  asm volatile("" ::"s"(nitems), "s"(item.x), "s"(item.y));
  if (want >= nitems) return;
  const int s = (int)(item.x >> 16);
  const int chunk = (int)(item.x & 0xffffu);
  if (s >= num_seqs) return;
  const int L = clamp_context(item.y, max_ctx, cap_tokens);
  if (L <= 0) return;
  const int nblk = (L + BS - 1) / BS;
  const int nchunks = (nblk + PB * NW - 1) / (PB * NW);
  if (chunk >= nchunks) return;
  const int c_begin = chunk * PB * NW;
  const int c_nb = min(PB * NW, nblk - c_begin);
  const int b_begin = c_begin + (c_nb * wave) / NW;
  const int nb = c_begin + (c_nb * (wave + 1)) / NW - b_begin;
  if (nb <= 0) return;
  const uint32_t my_bt =
      lane < nb ? block_tables[(int64_t)s * block_table_stride + b_begin + lane] : 0u;
  const int64_t head_off = (int64_t)j * head_stride_v + lane;
  const int n = 2 * nb * KPL;  // loads per lane: K tiles, then V tiles
  auto load = [&](int i0, uint4(&buf)[NV]) {
#pragma unroll
    for (int u = 0; u < NV; ++u) {
      const int i = i0 + u;
      if (i < n) {
        const int tile = i / KPL;
        const bool v = tile >= nb;
        const int bi = v ? tile - nb : tile;
        const uint32_t phys = (uint32_t)__builtin_amdgcn_readlane((int)my_bt, bi);
        const int64_t pb = (int64_t)phys < num_blocks ? (int64_t)phys : 0;
        buf[u] = tile_load((v ? value_cache : key_cache) + pb * block_stride_v + head_off +
                           64 * (i % KPL));
      }
    }
  };
  uint32_t acc = 0;
  auto fold = [&](int i0, const uint4(&buf)[NV]) {
#pragma unroll
    for (int u = 0; u < NV; ++u)
      if (i0 + u < n) acc ^= buf[u].x ^ buf[u].y ^ buf[u].z ^ buf[u].w;
  };
  uint4 a[NV], b[NV];
  load(0, a);
  load(NV, b);
  for (int i = 0; i < n; i += 2 * NV) {
    fold(i, a);
    load(i + 2 * NV, a);
    fold(i + NV, b);
    load(i + 3 * NV, b);
  }
  if (acc == magic) sink[0] = acc;
}

template <int BS, int KPL>
hipError_t launch_read_t(const void* kc, const void* vc, const uint32_t* bt, int32_t bts,
                         int32_t max_ctx, int32_t num_seqs, const CacheGeom& g, int elem_bytes,
                         const DecodeWorkspace& ws, uint32_t magic, uint32_t* sink,
                         hipStream_t stream) {
  const int max_chunks = max(1, (max_ctx + kDecodeChunk - 1) / kDecodeChunk);
  const int64_t units = (int64_t)num_seqs * max_chunks * g.num_kv_heads;
  const int64_t per_vec = 16 / elem_bytes;
  hipLaunchKernelGGL((paged_read_kernel<BS, KPL>), dim3((unsigned)units), dim3(64 * kRowsWaves),
                     0, stream, static_cast<const uint4*>(kc), static_cast<const uint4*>(vc), bt,
                     bts, g.num_kv_heads, g.num_blocks, g.block_stride / per_vec,
                     g.head_stride / per_vec, ws.items, ws.queue, num_seqs, max_ctx,
                     bts * g.block_size, magic, sink);
  return hipGetLastError();
}

}  // namespace

bool paged_read_supported(int cache_dtype, int head_dim, int block_size) {
  const int eb = cache_dtype == VPA_DTYPE_FP8_E4M3 ? 1
                 : (cache_dtype == VPA_DTYPE_BF16 || cache_dtype == VPA_DTYPE_F16) ? 2 : 0;
  if (eb == 0 || !(head_dim == 64 || head_dim == 128) ||
      !cache_kernels_supported(cache_dtype, head_dim, block_size))
    return false;
  const int tile = head_dim * block_size * eb;
  return tile % 1024 == 0 && tile / 1024 <= 8;
}

hipError_t launch_paged_read(int cache_dtype, const void* key_cache, const void* value_cache,
                             const uint32_t* block_tables, int32_t block_table_stride,
                             int32_t max_context_len, int32_t num_seqs, const CacheGeom& g,
                             const DecodeWorkspace& ws, uint32_t magic, uint32_t* sink,
                             hipStream_t stream) {
  const int eb = cache_dtype == VPA_DTYPE_FP8_E4M3 ? 1 : 2;
  const int kpl = g.head_dim * g.block_size * eb / 1024;
#define VPA_READ_CASE(BSV, K)                                                             \
  if (g.block_size == BSV && kpl == K)                                                     \
    return launch_read_t<BSV, K>(key_cache, value_cache, block_tables, block_table_stride, \
                                 max_context_len, num_seqs, g, eb, ws, magic, sink, stream);
  VPA_READ_CASE(8, 1) VPA_READ_CASE(8, 2) VPA_READ_CASE(16, 1) VPA_READ_CASE(16, 2)
  VPA_READ_CASE(16, 4) VPA_READ_CASE(32, 1) VPA_READ_CASE(32, 2) VPA_READ_CASE(32, 4)
  VPA_READ_CASE(32, 8)
#undef VPA_READ_CASE
  return hipErrorInvalidValue;
}

hipError_t launch_decode_plan(int dtype, const uint32_t* context_lens, int32_t max_context_len,
                              int32_t block_table_stride, int32_t num_seqs, const CacheGeom& g,
                              const DecodeWorkspace& ws, hipStream_t stream) {
  const bool rows = decode_uses_rows_kernel(dtype, g.head_dim, g.block_size);
  if (!rows || num_seqs == 0) return hipSuccess;
  hipLaunchKernelGGL(decode_plan_kernel, dim3(1), dim3(1024), 0, stream, context_lens, num_seqs,
                     max_context_len, block_table_stride * g.block_size, kDecodeChunk, ws.items,
                     ws.queue);
  return hipGetLastError();
}

bool decode_supported(int dtype, int head_dim, int block_size, int group) {
  const int x = dtype == VPA_DTYPE_F32 ? 4 : 8;
  return dtype != VPA_DTYPE_FP8_E4M3 && cache_kernels_supported(dtype, head_dim, block_size) &&
         (head_dim * block_size / x) % 64 == 0 && group >= 1;
}

int decode_kernel_group(int group) { return group % 4 == 0 ? 4 : group % 2 == 0 ? 2 : 1; }

// kFusedAppendMaxSeqs, or VPA_FUSED_APPEND_MAX_SEQS from the environment
// (read once): the crossover depends on the lengths and the part.
int fused_append_max_seqs() {
  static const int v = [] {
    const char* e = getenv("VPA_FUSED_APPEND_MAX_SEQS");
    if (e == nullptr || *e == '\0') return kFusedAppendMaxSeqs;
    char* end = nullptr;
    const long n = strtol(e, &end, 10);
    return (end != e && *end == '\0' && n >= 0 && n <= 65535) ? (int)n : kFusedAppendMaxSeqs;
  }();
  return v;
}

bool decode_fuses_append(int dtype, int cache_dtype, int head_dim, int block_size,
                         int num_seqs, int group) {
  return cache_dtype == dtype && decode_uses_rows_kernel(dtype, head_dim, block_size) &&
         fused_append_shape(head_dim, block_size) && num_seqs <= fused_append_max_seqs() &&
         decode_kernel_group(group) == group;
}

bool decode_uses_rows_kernel(int dtype, int head_dim, int block_size) {
  if (!(dtype == VPA_DTYPE_BF16 || dtype == VPA_DTYPE_F16)) return false;
  if (!cache_kernels_supported(dtype, head_dim, block_size)) return false;
  const int units = head_dim * block_size / 8;  // 16-byte units of a 16-bit tile
  return units % 64 == 0 && units / 64 <= 8;
}

bool decode_f32_fp8_shape(int head_dim, int block_size) {
  // (tiles of at most 6 KiB: the 8 KiB one, head dim 256 at 32-token
  // blocks, would not fit the generic kernel's registers with its dequantised
  // elements)
  const int units = head_dim * block_size / 16;
  return cache_kernels_supported(VPA_DTYPE_FP8_E4M3, head_dim, block_size) && block_size >= 16 &&
         units % 64 == 0 && units / 64 <= 6;
}

bool decode_fp8_shape(int head_dim, int block_size) {
  if (!cache_kernels_supported(VPA_DTYPE_FP8_E4M3, head_dim, block_size)) return false;
  // the two 16-bit tiles the rows kernel does not take: the generic kernel
  if (block_size == 32 && (head_dim == 192 || head_dim == 256)) return true;
  if (!decode_uses_rows_kernel(VPA_DTYPE_BF16, head_dim, block_size)) return false;
  // a whole number of 1 KiB loads per fp8 tile (at 8-token blocks a value
  // unit holds two dims: head dims 128 and 256)
  return block_size == 8 ? head_dim % 128 == 0 : (head_dim * block_size / 16) % 64 == 0;
}

namespace {
struct WorkspacePlan {
  size_t part_out, part_stat, items, queue, total;
  int max_parts;
};
// Pieces of the decode scratch for split-K partitions of part_tokens tokens
// (the caller workspace uses the smallest partition any kernel takes, so its
// size depends on the sizes only; the tight layout uses the partition of
// the kernel a configuration runs).
WorkspacePlan plan_workspace(int num_seqs, int num_heads, int head_dim, int max_context_len,
                             int part_tokens) {
  auto up = [](size_t b) { return (b + 255) & ~(size_t)255; };
  WorkspacePlan w{};
  w.max_parts = (max_context_len + part_tokens - 1) / part_tokens;
  const size_t rows = w.max_parts > 1 ? (size_t)num_seqs * (size_t)num_heads * (size_t)w.max_parts : 0;
  w.part_out = up(rows * (size_t)(head_dim + 32) * sizeof(float));
  w.part_stat = up(rows * sizeof(float));
  w.items = up((size_t)num_seqs * (size_t)(w.max_parts > 1 ? w.max_parts : 1) * sizeof(uint2));
  w.queue = 256;
  w.total = w.part_out + 2 * w.part_stat + w.items + w.queue;
  return w;
}
}  // namespace

int decode_part_tokens(int dtype, int head_dim, int block_size) {
  return decode_uses_rows_kernel(dtype, head_dim, block_size) ? kDecodeChunk : kPT;
}

size_t decode_workspace_bytes(int num_seqs, int num_heads, int head_dim, int max_context_len,
                              int part_tokens) {
  if (num_seqs <= 0 || num_heads <= 0 || head_dim <= 0 || max_context_len < 0 ||
      part_tokens <= 0)
    return 0;
  return plan_workspace(num_seqs, num_heads, head_dim, max_context_len, part_tokens).total;
}

DecodeWorkspace carve_decode_workspace(void* base, int num_seqs, int num_heads, int head_dim,
                                       int max_context_len, int part_tokens) {
  DecodeWorkspace ws{};
  const WorkspacePlan w =
      plan_workspace(num_seqs, num_heads, head_dim, max_context_len, part_tokens);
  ws.max_parts = w.max_parts;
  char* p = static_cast<char*>(base);
  ws.part_out = reinterpret_cast<float*>(p);
  p += w.part_out;
  ws.part_max = reinterpret_cast<float*>(p);
  p += w.part_stat;
  ws.part_sum = reinterpret_cast<float*>(p);
  p += w.part_stat;
  ws.items = reinterpret_cast<uint2*>(p);
  p += w.items;
  ws.queue = reinterpret_cast<uint32_t*>(p);
  return ws;
}

hipError_t launch_paged_decode(int dtype, int cache_dtype, void* out, const void* query,
                               const void* key_cache, const void* value_cache,
                               const uint32_t* block_tables, int32_t block_table_stride,
                               const uint32_t* context_lens, int32_t max_context_len,
                               float scale, const float* k_scale, const float* v_scale,
                               int32_t num_seqs, int32_t num_heads, const CacheGeom& g,
                               const DecodeWorkspace& ws, hipStream_t stream,
                               const DecodeAppend* append) {
  // G query heads per kv head run as kv_rep = G / group replicas of each kv
  // head, group (1, 2 or 4) query heads each: every replica reads its kv
  // head's tiles (kv_rep times the K/V bytes of one pass, for G of 8 or more)
  const int group = decode_kernel_group(num_heads / g.num_kv_heads);
  CacheGeom gv = g;
  gv.kv_rep = num_heads / g.num_kv_heads / group;
  gv.num_kv_heads = g.num_kv_heads * gv.kv_rep;
  if (cache_dtype == VPA_DTYPE_FP8_E4M3)
    return dispatch_decode_fp8(dtype, g.head_dim, g.block_size, group, out, query, key_cache,
                               value_cache, block_tables, block_table_stride, context_lens,
                               max_context_len, scale, num_seqs, num_heads, gv, ws, stream,
                               k_scale, v_scale, append);
  return dispatch_decode(dtype, g.head_dim, g.block_size, group, out, query, key_cache,
                         value_cache, block_tables, block_table_stride, context_lens,
                         max_context_len, scale, num_seqs, num_heads, gv, ws, stream, k_scale,
                         v_scale, append);
}

}  // namespace vpa
