// Chunked-prefill attention over the paged cache on the vector ALUs: the
// configurations the MFMA kernel (prefill_kernels.hip) does not take. f32
// queries over f32 or fp8 caches (the Metal prefill's `float` and
// `float, uint8_t` instances, vasr-paged-attn/src/metal/kernels/
// prefill_paged_attn.metal:1606, 1610, dispatched for F32 at
// vasr-paged-attn/src/metal/kernels/mod.rs:119-137), any number of query
// heads per kv head (the Metal dispatch takes q_per_kv as a grid dimension,
// mod.rs:145-283), and the 16-bit head-dim / block-size pairs without a
// whole number of 1 KiB DMAs per tile.
//
// Decode (paged_attention) runs the head-dim / block-size pairs its own
// kernels do not take on this kernel too, with one query per sequence (no
// cu_seqlens_q), causal, over the whole context, and denom_eps 1e-6.
//
// Semantics are the MFMA kernel's: query i of a sequence with n queries and
// L keys sees keys t <= i + L - n when causal (bottom-right alignment, the
// cached-causal mask of vasr-models/src/model/attention.rs:78-149), every key
// otherwise; keys in blocks outside the pool are skipped; out = sum p v /
// (sum p + denom_eps) with p = exp(s - max), 0 for a row that sees no key.
// An fp8 element is read as f32(E4M3FN(byte) * scale) rounded to the query
// type (prefill_paged_attn.metal:764-769, 797-800).
//
// Work unit (one workgroup of 256 threads): 16 consecutive (position, head)
// rows of one (sequence, kv head), one row per 16-lane group (rows run over
// the G query heads of the group fastest, so any G works). Per 32-key tile:
//   load: K and V of the tile to LDS as f32 (16-byte loads of whole key
//     units and of 4-token value runs, dequantised / widened once);
//   scores: lane l of a group forms the dot products of keys l and l + 16
//     with its row (float4 LDS reads, q and K rows padded so the 16 lanes
//     and the 4 groups of a wave hit distinct banks);
//   online softmax per row in f32 (max and sum over the group's lanes with
//     shuffles; the reference max is the true running max);
//   P.V: lane l sums the tile's contribution to 4-dim chunks l, l + 16, ...
//     of its row's output and adds it to the rescaled running sum.
// The dot products keep four partial sums and the P.V sums run per tile, so
// no f32 rounding chain is longer than a quarter of the head dim or one
// tile's keys (at head dim 256 a single running sum put elements near zero
// past the f32 bound against the fp64 oracle).
// Measured on c4's lengths with 24 query heads (3 per kv head): 14.6 ms in
// f32, 13.3 ms in bf16 (23-25 TFLOP/s); the MFMA kernel runs the bf16 c4
// shape at ~310 us.
#include <type_traits>

#include "vpa_device.h"
#include "vpa_internal.h"

namespace vpa {
namespace {

constexpr int kVRows = 16;       // rows per workgroup (one per 16-lane group)
constexpr int kVKeys = 32;       // keys per tile
constexpr int kVThreads = 256;
static_assert(kVRows * 16 == kVThreads, "one 16-lane group per row");

// One fp8 (E4M3FN) byte as f32 (exact), through gfx950's conversion to
// bf16.
__device__ __forceinline__ float fp8_byte_to_f32(uint32_t b) {
  return bf16_bits_to_f32(fp8x2_to_pk<bf16_t>(b & 0xffu, false) & 0xffffu);
}

// f32 rounded to T and widened back (the query type of the dequantised
// cache element)
template <typename T>
__device__ __forceinline__ float round_to(float v) {
  if constexpr (std::is_same_v<T, bf16_t>) return bf16_bits_to_f32(f32_to_bf16_bits(v));
  else if constexpr (std::is_same_v<T, f16_t>) return f16_bits_to_f32(f32_to_f16_bits(v));
  else return v;
}

// Element e (0..7) of a 16-byte vector of 16-bit values as f32
template <typename C>
__device__ __forceinline__ float half_elem(const uint4& v, int e) {
  const uint32_t w = e < 2 ? v.x : e < 4 ? v.y : e < 6 ? v.z : v.w;
  const uint32_t h = (e & 1) ? (w >> 16) : (w & 0xffffu);
  if constexpr (std::is_same_v<C, bf16_t>) return bf16_bits_to_f32(h);
  else return f16_bits_to_f32((uint16_t)h);
}

__device__ __forceinline__ float group16_max(float v) {
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 16));
  return v;
}
__device__ __forceinline__ float group16_sum(float v) {
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) v += __shfl_xor(v, o, 16);
  return v;
}

// T: query / output type (float, bf16_t, f16_t); C: cache element type (T or
// fp8_t); D: head_dim. Block size is a runtime power of two (8, 16, 32).
template <typename T, typename C, int D>
__global__ __launch_bounds__(kVThreads) void prefill_paged_vector_kernel(
    T* __restrict__ out, const T* __restrict__ query, const C* __restrict__ key_cache,
    const C* __restrict__ value_cache, const uint32_t* __restrict__ block_tables,
    int32_t block_table_stride, const uint32_t* __restrict__ cu_seqlens_q,
    const uint32_t* __restrict__ context_lens, int32_t max_query_len, int32_t max_kv_len,
    int64_t total_query_rows, float scale_log2, float denom_eps, int32_t causal,
    int32_t num_heads, int32_t num_kv_heads, int32_t group, int32_t block_size_log2,
    int64_t num_blocks, int64_t block_stride, int64_t head_stride, int32_t row_tiles,
    const float* __restrict__ k_scale, const float* __restrict__ v_scale) {
  constexpr bool kF8 = std::is_same_v<C, fp8_t>;
  static_assert(kF8 || std::is_same_v<C, T>, "cache type is the query type or fp8");
  static_assert(D % 16 == 0, "head_dim");
  constexpr int X = pack_x<C>();        // cache elements per 16-byte unit
  constexpr int NCH = (D / 4 + 15) / 16;  // 4-dim output chunks per lane
  constexpr int QP = D + 4;             // padded row pitch of q and K in LDS (floats)
  constexpr int PP = kVKeys + 4;        // padded row pitch of the probabilities

  __shared__ __align__(16) float s_q[kVRows][QP];
  __shared__ __align__(16) float s_k[kVKeys][QP];
  __shared__ __align__(16) float s_v[kVKeys][D];
  __shared__ __align__(16) float s_p[kVRows][PP];

  const int tid = threadIdx.x;
  const int r = tid >> 4;     // this group's row
  const int l = tid & 15;     // lane in the group
  const int BS = 1 << block_size_log2;
  // consecutive workgroups: kv heads, then the row tiles of one sequence
  const int j = (int)(blockIdx.x % (uint32_t)num_kv_heads);
  const int rest = (int)(blockIdx.x / (uint32_t)num_kv_heads);
  const int s = rest / row_tiles;
  const int rt = rest % row_tiles;

  // (no cu_seqlens_q: one query per sequence, row s — the decode form)
  const uint32_t qa = cu_seqlens_q != nullptr ? cu_seqlens_q[s] : (uint32_t)s;
  const uint32_t qb = cu_seqlens_q != nullptr ? cu_seqlens_q[s + 1] : (uint32_t)s + 1u;
  int q_len = qb > qa ? (int)min(qb - qa, (uint32_t)max_query_len) : 0;
  if ((int64_t)qa >= total_query_rows) q_len = 0;
  else q_len = (int)min((int64_t)q_len, total_query_rows - (int64_t)qa);
  const int k_len = (int)min(context_lens[s], (uint32_t)max_kv_len);
  const int64_t row0 = (int64_t)rt * kVRows;  // first (position, head) row of the tile
  if (row0 >= (int64_t)q_len * group) return;  // whole workgroup past this sequence's rows

  const int64_t ri = row0 + r;
  const int pos = (int)(ri / group);
  const int head = j * group + (int)(ri % group);
  const bool row_ok = pos < q_len;
  const int shift = k_len - q_len;  // bottom-right causal alignment
  const int limit = causal ? pos + shift : k_len - 1;  // last key the row sees
  const int last_pos = (int)min((row0 + kVRows - 1) / group, (int64_t)q_len - 1);
  const int n_keys = max(0, causal ? min(k_len, last_pos + shift + 1) : k_len);

  float ks = 1.f, vs = 1.f;
  if constexpr (kF8) {
    ks = *k_scale;
    vs = *v_scale;
  }

  // this row's query, widened to f32
  {
    const T* qrow = query + (((int64_t)qa + pos) * num_heads + head) * D;
    for (int d = l; d < D; d += 16) s_q[r][d] = row_ok ? load_as_f32(qrow + d) : 0.f;
  }

  const C* kbase = key_cache + (int64_t)j * head_stride;
  const C* vbase = value_cache + (int64_t)j * head_stride;
  const uint32_t* bt = block_tables + (int64_t)s * block_table_stride;

  float4 acc[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) acc[c] = make_float4(0.f, 0.f, 0.f, 0.f);
  float m = -INFINITY;  // the row's running max (log2 units)
  float lsum = 0.f;     // sum of probabilities against m (replicated over the group)

  for (int k0 = 0; k0 < n_keys; k0 += kVKeys) {
    __syncthreads();  // the previous tile's K / V / P are consumed
    // K units: (key k, X-dim chunk c); V runs: (dim d, 4 tokens)
    constexpr int KU = kVKeys * (D / X);
    for (int i = tid; i < KU; i += kVThreads) {
      const int k = i / (D / X), c = i - k * (D / X);
      const int t = k0 + k;
      float v[X];
      bool ok = t < k_len;
      uint32_t blk = 0;
      if (ok) {
        blk = bt[t >> block_size_log2];
        ok = (int64_t)blk < num_blocks;
      }
      if (ok) {
        const uint4 u = *reinterpret_cast<const uint4*>(
            kbase + (int64_t)blk * block_stride + ((int64_t)c * BS + (t & (BS - 1))) * X);
        if constexpr (kF8) {
          const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
          for (int e = 0; e < 16; ++e)
            v[e] = round_to<T>(fp8_byte_to_f32(w[e / 4] >> (8 * (e % 4))) * ks);
        } else if constexpr (std::is_same_v<C, float>) {
          v[0] = __uint_as_float(u.x);
          v[1] = __uint_as_float(u.y);
          v[2] = __uint_as_float(u.z);
          v[3] = __uint_as_float(u.w);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = half_elem<C>(u, e);
        }
      } else {
#pragma unroll
        for (int e = 0; e < X; ++e) v[e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < X; ++e) s_k[k][c * X + e] = v[e];
    }
    constexpr int VU = D * (kVKeys / 4);
    for (int i = tid; i < VU; i += kVThreads) {
      const int d = i / (kVKeys / 4), q4 = i - d * (kVKeys / 4);
      const int t = k0 + 4 * q4;  // 4 tokens of one block (blocks hold 8..32)
      float v[4] = {0.f, 0.f, 0.f, 0.f};
      if (t < k_len) {
        const uint32_t blk = bt[t >> block_size_log2];
        if ((int64_t)blk < num_blocks) {
          const C* src = vbase + (int64_t)blk * block_stride + (int64_t)d * BS + (t & (BS - 1));
          if constexpr (kF8) {
            const uint32_t w = *reinterpret_cast<const uint32_t*>(src);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = round_to<T>(fp8_byte_to_f32(w >> (8 * e)) * vs);
          } else if constexpr (std::is_same_v<C, float>) {
            const float4 f = *reinterpret_cast<const float4*>(src);
            v[0] = f.x;
            v[1] = f.y;
            v[2] = f.z;
            v[3] = f.w;
          } else {
            const uint2 h = *reinterpret_cast<const uint2*>(src);
            const uint4 u = make_uint4(h.x, h.y, 0u, 0u);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = half_elem<C>(u, e);
          }
        }
      }
      // tokens past the context or in absent blocks hold 0 (stale slots may
      // hold NaN, and 0 * NaN would poison the row)
#pragma unroll
      for (int e = 0; e < 4; ++e) s_v[4 * q4 + e][d] = t + e < k_len ? v[e] : 0.f;
    }
    __syncthreads();

    // scores of keys l and l + 16 against this row: four partial sums per
    // key (dims 4i + c), added pairwise at the end (shorter rounding chains
    // than one running sum over the head dim)
    float4 a0 = make_float4(0.f, 0.f, 0.f, 0.f), a1 = a0;
#pragma unroll 8
    for (int d = 0; d < D; d += 4) {
      const float4 q4 = *reinterpret_cast<const float4*>(&s_q[r][d]);
      const float4 x0 = *reinterpret_cast<const float4*>(&s_k[l][d]);
      const float4 x1 = *reinterpret_cast<const float4*>(&s_k[l + 16][d]);
      a0.x = fmaf(q4.x, x0.x, a0.x);
      a0.y = fmaf(q4.y, x0.y, a0.y);
      a0.z = fmaf(q4.z, x0.z, a0.z);
      a0.w = fmaf(q4.w, x0.w, a0.w);
      a1.x = fmaf(q4.x, x1.x, a1.x);
      a1.y = fmaf(q4.y, x1.y, a1.y);
      a1.z = fmaf(q4.z, x1.z, a1.z);
      a1.w = fmaf(q4.w, x1.w, a1.w);
    }
    const float d0 = (a0.x + a0.y) + (a0.z + a0.w);
    const float d1 = (a1.x + a1.y) + (a1.z + a1.w);
    auto visible = [&](int t) {
      if (t >= k_len || t > limit) return false;
      return (int64_t)bt[t >> block_size_log2] < num_blocks;
    };
    const float s0 = visible(k0 + l) ? d0 * scale_log2 : -INFINITY;
    const float s1 = visible(k0 + l + 16) ? d1 * scale_log2 : -INFINITY;
    const float m_new = fmaxf(m, group16_max(fmaxf(s0, s1)));
    float p0 = 0.f, p1 = 0.f, alpha = 1.f;
    if (m_new != -INFINITY) {
      alpha = m == -INFINITY ? 0.f : exp2f(m - m_new);
      p0 = s0 == -INFINITY ? 0.f : exp2f(s0 - m_new);
      p1 = s1 == -INFINITY ? 0.f : exp2f(s1 - m_new);
    }
    lsum = lsum * alpha + group16_sum(p0 + p1);
    m = m_new;
    s_p[r][l] = p0;
    s_p[r][l + 16] = p1;
    __builtin_amdgcn_s_waitcnt(0xc07f);  // this wave's LDS writes of P are done
    __builtin_amdgcn_wave_barrier();
    // P.V over the tile into a tile sum, added to the rescaled running sum
    // (so no rounding chain runs over more than one tile's keys): lane l owns
    // 4-dim chunks l, l + 16, ...
    float4 ta[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) ta[c] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 4
    for (int k4 = 0; k4 < kVKeys; k4 += 4) {
      const float4 p4 = *reinterpret_cast<const float4*>(&s_p[r][k4]);
      const float pk[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
          const int ch = l + 16 * c;
          if (ch < D / 4) {
            const float4 v4 = *reinterpret_cast<const float4*>(&s_v[k4 + e][4 * ch]);
            ta[c].x = fmaf(pk[e], v4.x, ta[c].x);
            ta[c].y = fmaf(pk[e], v4.y, ta[c].y);
            ta[c].z = fmaf(pk[e], v4.z, ta[c].z);
            ta[c].w = fmaf(pk[e], v4.w, ta[c].w);
          }
        }
      }
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      acc[c].x = fmaf(acc[c].x, alpha, ta[c].x);
      acc[c].y = fmaf(acc[c].y, alpha, ta[c].y);
      acc[c].z = fmaf(acc[c].z, alpha, ta[c].z);
      acc[c].w = fmaf(acc[c].w, alpha, ta[c].w);
    }
  }

  if (!row_ok) return;
  // the sums are relative to the row's true max, so the epsilon is added as
  // it stands; a row that sees no key gives 0
  const float inv = lsum > 0.f ? 1.f / (lsum + denom_eps) : 0.f;
  T* orow = out + (((int64_t)qa + pos) * num_heads + head) * D;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int ch = l + 16 * c;
    if (ch < D / 4) {
      store_from_f32<T>(orow + 4 * ch + 0, acc[c].x * inv);
      store_from_f32<T>(orow + 4 * ch + 1, acc[c].y * inv);
      store_from_f32<T>(orow + 4 * ch + 2, acc[c].z * inv);
      store_from_f32<T>(orow + 4 * ch + 3, acc[c].w * inv);
    }
  }
}

template <typename T, typename C, int D>
hipError_t launch_vector_t(void* out, const void* query, const void* kc, const void* vc,
                           const uint32_t* bt, int32_t bts, const uint32_t* cu,
                           const uint32_t* cl, int32_t num_seqs, int32_t max_query_len,
                           int32_t max_kv_len, int64_t total_query_rows, float scale,
                           float denom_eps, int32_t causal, int32_t num_heads, const CacheGeom& g,
                           const float* k_scale, const float* v_scale, hipStream_t stream) {
  const int group = num_heads / g.num_kv_heads;
  const int64_t row_tiles = ((int64_t)max_query_len * group + kVRows - 1) / kVRows;
  const int64_t grid = (int64_t)num_seqs * row_tiles * g.num_kv_heads;
  if (grid == 0) return hipSuccess;
  int bs_log2 = 0;
  while ((1 << bs_log2) < g.block_size) ++bs_log2;
  hipLaunchKernelGGL((prefill_paged_vector_kernel<T, C, D>), dim3((uint32_t)grid),
                     dim3(kVThreads), 0, stream, static_cast<T*>(out),
                     static_cast<const T*>(query), static_cast<const C*>(kc),
                     static_cast<const C*>(vc), bt, bts, cu, cl, max_query_len, max_kv_len,
                     total_query_rows, scale * 1.4426950408889634f, denom_eps, causal, num_heads,
                     g.num_kv_heads, group, bs_log2, g.num_blocks, g.block_stride, g.head_stride,
                     (int32_t)row_tiles, k_scale, v_scale);
  return hipGetLastError();
}

template <typename T, typename C, typename... A>
hipError_t vector_dim(int d, A... args) {
  switch (d) {
    case 64:
      return launch_vector_t<T, C, 64>(args...);
    case 96:
      return launch_vector_t<T, C, 96>(args...);
    case 128:
      return launch_vector_t<T, C, 128>(args...);
    case 192:
      return launch_vector_t<T, C, 192>(args...);
    case 256:
      return launch_vector_t<T, C, 256>(args...);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace

bool prefill_vector_supported(int dtype, int cache_dtype, int head_dim, int block_size) {
  const bool qt = dtype == VPA_DTYPE_F32 || dtype == VPA_DTYPE_BF16 || dtype == VPA_DTYPE_F16;
  const bool ct = cache_dtype == dtype || cache_dtype == VPA_DTYPE_FP8_E4M3;
  const bool dim = head_dim == 64 || head_dim == 96 || head_dim == 128 || head_dim == 192 ||
                   head_dim == 256;
  const bool blk = block_size == 8 || block_size == 16 || block_size == 32;
  return qt && ct && dim && blk;
}

int64_t prefill_vector_workgroups(int32_t num_seqs, int32_t max_query_len, int32_t group,
                                  int32_t num_kv_heads) {
  return (int64_t)num_seqs * (((int64_t)max_query_len * group + kVRows - 1) / kVRows) *
         num_kv_heads;
}

hipError_t launch_prefill_vector(int dtype, int cache_dtype, void* out, const void* query,
                                 const void* key_cache, const void* value_cache,
                                 const uint32_t* block_tables, int32_t block_table_stride,
                                 const uint32_t* cu_seqlens_q, const uint32_t* context_lens,
                                 int32_t num_seqs, int32_t max_query_len, int32_t max_kv_len,
                                 int64_t total_query_rows, float scale, float denom_eps,
                                 int32_t causal, int32_t num_heads, const CacheGeom& g,
                                 const float* k_scale, const float* v_scale,
                                 hipStream_t stream) {
  const bool f8 = cache_dtype == VPA_DTYPE_FP8_E4M3;
#define VPA_VEC_ARGS                                                                            \
  g.head_dim, out, query, key_cache, value_cache, block_tables, block_table_stride,            \
      cu_seqlens_q, context_lens, num_seqs, max_query_len, max_kv_len, total_query_rows, scale, \
      denom_eps, causal, num_heads, g, k_scale, v_scale, stream
  if (dtype == VPA_DTYPE_F32)
    return f8 ? vector_dim<float, fp8_t>(VPA_VEC_ARGS) : vector_dim<float, float>(VPA_VEC_ARGS);
  if (dtype == VPA_DTYPE_BF16)
    return f8 ? vector_dim<bf16_t, fp8_t>(VPA_VEC_ARGS)
              : vector_dim<bf16_t, bf16_t>(VPA_VEC_ARGS);
  if (dtype == VPA_DTYPE_F16)
    return f8 ? vector_dim<f16_t, fp8_t>(VPA_VEC_ARGS) : vector_dim<f16_t, f16_t>(VPA_VEC_ARGS);
#undef VPA_VEC_ARGS
  return hipErrorInvalidValue;
}

}  // namespace vpa
