// Chunked-prefill attention read straight from the paged KV cache (gfx950
// MFMA).
//
// The reference's packed paged prefill appends the new K/V with
// reshape_and_cache, gathers every sequence's cached tokens into packed
// [sum L, KVH, D] tensors (gather_kv_cache, vasr-models/src/model/
// thinker_text.rs:1344-1352) and runs flash varlen attention over them
// (thinker_text.rs:1353-1365 -> attention.rs:694-738 -> flash_attn_varlen,
// attention.rs:554-664). Causal masking is bottom-right aligned: query i of
// a sequence with n queries and L keys sees keys t <= i + L - n, which is the
// cached-causal mask of attention.rs:78-149. This kernel fuses the gather:
// K and V tiles go from the paged cache through LDS into the MFMA operands,
// so the gathered copy never exists in HBM.
//
// Work unit (one workgroup of 4 waves): one (sequence, kv head, tile of
// 128 / G query positions); wave w owns 32 query rows = 32 / G positions x
// G heads of the GQA group, so all G heads share every K/V tile.
//
// Per 32-key tile, S^T = K . Q^T with v_mfma_f32_32x32x16 (A = K rows from
// LDS, B = this lane's query row held in registers). In the 32x32 result,
// lane l owns query column l % 32 and 16 of the 32 keys, so the online
// softmax state (running max m, partial sum l) is per lane and needs one
// cross-half exchange per tile. O^T += V^T . P^T then takes P^T straight
// from the S^T accumulator: MFMA sums over k in any order as long as the A
// and B operands agree, so V^T's k slots are read from LDS in the key order
// the accumulator already has (keys 4h..4h+3 and 8+4h..8+4h+3 of each
// 16-key step for lane half h). The probabilities are rounded to the cache
// type for the MFMA; the row sums use the unrounded values. The output is
// acc / sum without an epsilon, as flash attention computes it.
#include "vpa_device.h"
#include "vpa_internal.h"

namespace vpa {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

template <typename T>
__device__ __forceinline__ f32x16_t mfma32x32x16(const uint4& a, const uint4& b,
                                                 const f32x16_t& c);
template <>
__device__ __forceinline__ f32x16_t mfma32x32x16<bf16_t>(const uint4& a, const uint4& b,
                                                         const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x16_t mfma32x32x16<f16_t>(const uint4& a, const uint4& b,
                                                        const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// max over lanes l and l ^ 32 (permlane32 swap of a value with itself
// returns both halves' values; one of the two results is the partner's)
__device__ __forceinline__ float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

#ifndef VPA_PREFILL_KEYS
#define VPA_PREFILL_KEYS 32
#endif
#ifndef VPA_PREFILL_COLS
#define VPA_PREFILL_COLS 1
#endif
constexpr int kPrefillKeys = VPA_PREFILL_KEYS;       // keys per LDS tile (32 or 64)
constexpr int kPrefillColGroups = VPA_PREFILL_COLS;  // 32-row query groups per wave (1 or 2)
#ifndef VPA_PREFILL_WAVES_PER_EU
#define VPA_PREFILL_WAVES_PER_EU 2
#endif
constexpr int kPrefillThreads = 256;

template <typename T, int D, int BS, int G>
__global__ __launch_bounds__(kPrefillThreads)
__attribute__((amdgpu_waves_per_eu(VPA_PREFILL_WAVES_PER_EU))) void prefill_paged_kernel(
    T* __restrict__ out, const T* __restrict__ query, const T* __restrict__ key_cache,
    const T* __restrict__ value_cache, const uint32_t* __restrict__ block_tables,
    int32_t block_table_stride, const uint32_t* __restrict__ cu_seqlens_q,
    const uint32_t* __restrict__ context_lens, int32_t num_seqs, int32_t max_query_len,
    int32_t max_kv_len, int64_t total_query_rows, float scale_log2, int32_t causal,
    int32_t num_heads, int32_t num_kv_heads, int64_t num_blocks, int64_t block_stride,
    int64_t head_stride, int32_t q_tiles) {
  constexpr int KT = kPrefillKeys;
  constexpr int CG = kPrefillColGroups;
  constexpr int X = 8;          // 16-bit elements per 16-byte key vector
  constexpr int ROWS = 32 * CG; // query rows per wave
  constexpr int PPW = ROWS / G; // query positions per wave
  constexpr int PPB = 4 * PPW;  // query positions per workgroup
  constexpr int KG = KT / 32;   // 32-key groups of a tile
  constexpr int KS = D / 16;    // k-steps of Q.K^T
  constexpr int DT = D / 32;    // 32-row tiles of O^T
  constexpr int VROW = KT + 4;  // LDS value row (elements): +8 bytes keeps b64 reads conflict-light
  constexpr int UPT = KT * D / 8 / kPrefillThreads;  // 16-byte units per thread per K / V tile
  constexpr int KSTEP = kPrefillThreads / KT;        // chunk stride of a thread's K units
  constexpr int OCT = KT / 8;                        // 8-key octets per value row
  constexpr int VSTEP = kPrefillThreads / OCT;       // dim stride of a thread's V units
  static_assert(BS >= 8 && (KT % BS == 0 || BS % KT == 0), "block size");
  static_assert((KT == 32 || KT == 64) && (CG == 1 || CG == 2) && UPT >= 1, "tile shape");
  static_assert(ROWS % G == 0 && D % 32 == 0, "rows");

  __shared__ __align__(16) uint4 s_k[2][D / X][KT];  // [chunk of 8 dims][key]
  __shared__ __align__(16) uint16_t s_v[2][D][VROW];  // [dim][key]
  __shared__ uint64_t s_valid[2];                     // keys of the tile that exist

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // consecutive workgroups: kv heads, then the query tiles of one sequence
  // (heaviest first), so the tiles of a (sequence, kv head) run together on
  // one XCD and share its K/V through L2
  const int j = (int)(blockIdx.x % (uint32_t)num_kv_heads);
  const int rest = (int)(blockIdx.x / (uint32_t)num_kv_heads);
  const int s = rest / q_tiles;
  const int qt = q_tiles - 1 - rest % q_tiles;

  const uint32_t qa = cu_seqlens_q[s], qb = cu_seqlens_q[s + 1];
  int q_len = qb > qa ? (int)min(qb - qa, (uint32_t)max_query_len) : 0;
  if ((int64_t)qa >= total_query_rows) q_len = 0;
  else q_len = (int)min((int64_t)q_len, total_query_rows - (int64_t)qa);
  const int k_len = (int)min(context_lens[s], (uint32_t)max_kv_len);

  const int p0 = qt * PPB;
  if (p0 >= q_len) return;  // whole workgroup: tile past this sequence's queries
  const int shift = k_len - q_len;  // bottom-right causal alignment
  const int wg_end = min(p0 + PPB, q_len);
  const int n_keys = max(0, causal ? min(k_len, wg_end + shift) : k_len);
  const int n_tiles = (n_keys + KT - 1) / KT;

  // this lane's query rows (one per column group; column of S^T and O^T)
  const int col = lane & 31;
  const int half = lane >> 5;
  const int wpos0 = p0 + wave * PPW;
  bool row_ok[CG];
  int64_t row[CG];
  int head[CG], limit[CG];
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    const int ri = cg * 32 + col;
    const int pos = wpos0 + ri % PPW;
    head[cg] = j * G + ri / PPW;
    row_ok[cg] = pos < q_len;
    row[cg] = (int64_t)qa + pos;
    limit[cg] = causal ? pos + shift : k_len - 1;  // last key the row sees
  }
  const int wave_end = min(wpos0 + PPW, q_len);
  const int wave_keys =
      wave_end <= wpos0 ? 0 : max(0, causal ? min(k_len, wave_end + shift) : k_len);
  const int wave_min_limit = causal ? wpos0 + shift : k_len - 1;

  uint4 qop[CG][KS];
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    const T* qrow = query + (row[cg] * num_heads + head[cg]) * D + 8 * half;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qop[cg][ks] =
          row_ok[cg] ? *reinterpret_cast<const uint4*>(qrow + 16 * ks) : make_uint4(0, 0, 0, 0);
  }

  f32x16_t o[CG][DT];
  float m[CG], lsum[CG];  // running max (log2 units) and this lane's share of the sum
#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    m[cg] = -INFINITY;
    lsum[cg] = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[cg][dt][e] = 0.f;
  }

  const T* kbase = key_cache + (int64_t)j * head_stride;
  const T* vbase = value_cache + (int64_t)j * head_stride;
  const uint32_t* bt = block_tables + (int64_t)s * block_table_stride;
  // loader roles: K units hold key tid % KT of chunks tid / KT + KSTEP i;
  // V units hold keys 8 (tid % OCT) .. +7 of dims tid / OCT + VSTEP i
  const int lk = tid % KT;
  const int lc = tid / KT;
  const int lo = tid % OCT;
  const int ld = tid / OCT;
  uint4 kreg[UPT], vreg[UPT];
  bool kvalid = false;

  auto load_tile = [&](int tt) {
    const int k0 = tt * KT;
    {
      const int key = k0 + lk;
      uint32_t phys = key < k_len ? bt[key / BS] : 0u;
      kvalid = key < k_len && (int64_t)phys < num_blocks;
      if (!kvalid) phys = 0u;  // read block 0 (in bounds); the key is masked
      const T* src = kbase + (int64_t)phys * block_stride + (key % BS) * X;
#pragma unroll
      for (int i = 0; i < UPT; ++i)
        kreg[i] = *reinterpret_cast<const uint4*>(src + (int64_t)(lc + KSTEP * i) * BS * X);
    }
    {
      const int key = k0 + 8 * lo;
      uint32_t phys = key < k_len ? bt[key / BS] : 0u;
      const bool ok = key < k_len && (int64_t)phys < num_blocks;
      if (!ok) phys = 0u;
      const T* src = vbase + (int64_t)phys * block_stride + (key % BS);
#pragma unroll
      for (int i = 0; i < UPT; ++i)
        vreg[i] = *reinterpret_cast<const uint4*>(src + (int64_t)(ld + VSTEP * i) * BS);
      // values of keys that do not exist are zeroed (stale cache contents
      // could be NaN, and 0 * NaN would poison the sum)
      const int nvalid = ok ? min(8, k_len - key) : 0;
      if (nvalid < 8) {
#pragma unroll
        for (int i = 0; i < UPT; ++i) {
          uint32_t w[4] = {vreg[i].x, vreg[i].y, vreg[i].z, vreg[i].w};
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (e >= nvalid) w[e / 2] &= (e & 1) ? 0x0000ffffu : 0xffff0000u;
          vreg[i] = make_uint4(w[0], w[1], w[2], w[3]);
        }
      }
    }
  };
  auto store_tile = [&](int b) {
#pragma unroll
    for (int i = 0; i < UPT; ++i) s_k[b][lc + KSTEP * i][lk] = kreg[i];
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      uint2* dst = reinterpret_cast<uint2*>(&s_v[b][ld + VSTEP * i][8 * lo]);
      dst[0] = make_uint2(vreg[i].x, vreg[i].y);
      dst[1] = make_uint2(vreg[i].z, vreg[i].w);
    }
    // lanes 0..KT-1 of wave 0 hold keys 0..KT-1 of the tile
    if (wave == 0) {
      const uint64_t bal = __ballot(kvalid);
      if (lane == 0) s_valid[b] = KT == 64 ? bal : (bal & 0xffffffffull);
    }
  };
  auto compute_tile = [&](int tt, int b) {
    const int k0 = tt * KT;
    if (k0 >= wave_keys) return;  // no row of this wave sees these keys
    const uint64_t vmask = s_valid[b];
    const bool full =
        vmask == (KT == 64 ? ~0ull : 0xffffffffull) && k0 + KT - 1 <= wave_min_limit;
    // S^T = K . Q^T: every K operand read from LDS feeds CG MFMAs
    f32x16_t sacc[KG][CG];
#pragma unroll
    for (int kg = 0; kg < KG; ++kg)
#pragma unroll
      for (int cg = 0; cg < CG; ++cg)
#pragma unroll
        for (int e = 0; e < 16; ++e) sacc[kg][cg][e] = 0.f;
#pragma unroll
    for (int kg = 0; kg < KG; ++kg)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const uint4 a = s_k[b][2 * ks + half][32 * kg + col];
#pragma unroll
        for (int cg = 0; cg < CG; ++cg)
          sacc[kg][cg] = mfma32x32x16<T>(a, qop[cg][ks], sacc[kg][cg]);
      }
    // online softmax per row; P^T operands straight from the accumulators
    uint4 pk[CG][2 * KG];
#pragma unroll
    for (int cg = 0; cg < CG; ++cg) {
      float sv[KG][16];
      float mx = -INFINITY;
#pragma unroll
      for (int kg = 0; kg < KG; ++kg)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = 32 * kg + 8 * (r / 4) + 4 * half + (r % 4);  // row of element r
          float v = sacc[kg][cg][r] * scale_log2;
          if (!full) v = (((vmask >> key) & 1ull) && k0 + key <= limit[cg]) ? v : -INFINITY;
          sv[kg][r] = v;
          mx = fmaxf(mx, v);
        }
      mx = max_xor32(mx);
      const float m_new = fmaxf(m[cg], mx);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = exp2f(m[cg] - m_use);
      float ps = 0.f;
#pragma unroll
      for (int kg = 0; kg < KG; ++kg)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          sv[kg][r] = exp2f(sv[kg][r] - m_use);
          ps += sv[kg][r];
        }
      lsum[cg] = lsum[cg] * alpha + ps;
      m[cg] = m_new;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[cg][dt][e] *= alpha;
#pragma unroll
      for (int k2 = 0; k2 < 2 * KG; ++k2) {
        const float* p = &sv[k2 / 2][8 * (k2 % 2)];
        pk[cg][k2] = make_uint4(pack2<T>(p[0], p[1]), pack2<T>(p[2], p[3]),
                                pack2<T>(p[4], p[5]), pack2<T>(p[6], p[7]));
      }
    }
    // O^T += V^T . P^T: k-step k2 covers keys 16 k2 + {4h..4h+3, 8+4h..8+4h+3}
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int k2 = 0; k2 < 2 * KG; ++k2) {
        const uint16_t* vr = &s_v[b][32 * dt + col][16 * k2 + 4 * half];
        const uint2 lo4 = *reinterpret_cast<const uint2*>(vr);
        const uint2 hi4 = *reinterpret_cast<const uint2*>(vr + 8);
        const uint4 a = make_uint4(lo4.x, lo4.y, hi4.x, hi4.y);
#pragma unroll
        for (int cg = 0; cg < CG; ++cg) o[cg][dt] = mfma32x32x16<T>(a, pk[cg][k2], o[cg][dt]);
      }
    }
  };

  if (n_tiles > 0) {
    load_tile(0);
    store_tile(0);
    __syncthreads();
    for (int tt = 0; tt < n_tiles; ++tt) {
      const int b = tt & 1;
      const bool more = tt + 1 < n_tiles;
      if (more) load_tile(tt + 1);  // in flight during this tile's MFMAs
      compute_tile(tt, b);
      if (more) store_tile(b ^ 1);
      __syncthreads();
    }
  }

#pragma unroll
  for (int cg = 0; cg < CG; ++cg) {
    const float total = sum_xor32(lsum[cg]);
    const float inv = total > 0.f ? 1.f / total : 0.f;  // a row that sees no key gives 0
    if (row_ok[cg]) {
      T* orow = out + (row[cg] * num_heads + head[cg]) * D;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d0 = 32 * dt + 8 * i + 4 * half;
          *reinterpret_cast<uint2*>(orow + d0) =
              make_uint2(pack2<T>(o[cg][dt][4 * i] * inv, o[cg][dt][4 * i + 1] * inv),
                         pack2<T>(o[cg][dt][4 * i + 2] * inv, o[cg][dt][4 * i + 3] * inv));
        }
    }
  }
}

template <typename T, int D, int BS, int G>
hipError_t launch_prefill_t(void* out, const void* query, const void* key_cache,
                            const void* value_cache, const uint32_t* block_tables,
                            int32_t block_table_stride, const uint32_t* cu_seqlens_q,
                            const uint32_t* context_lens, int32_t num_seqs,
                            int32_t max_query_len, int32_t max_kv_len, int64_t total_query_rows,
                            float scale, int32_t causal, int32_t num_heads, const CacheGeom& g,
                            hipStream_t stream) {
  constexpr int kPositions = 4 * 32 * kPrefillColGroups / G;
  const int q_tiles = (max_query_len + kPositions - 1) / kPositions;
  const int64_t grid = (int64_t)num_seqs * q_tiles * g.num_kv_heads;
  if (grid == 0) return hipSuccess;
  const float scale_log2 = scale * 1.4426950408889634f;
  hipLaunchKernelGGL((prefill_paged_kernel<T, D, BS, G>), dim3((uint32_t)grid),
                     dim3(kPrefillThreads), 0, stream, static_cast<T*>(out),
                     static_cast<const T*>(query), static_cast<const T*>(key_cache),
                     static_cast<const T*>(value_cache), block_tables, block_table_stride,
                     cu_seqlens_q, context_lens, num_seqs, max_query_len, max_kv_len,
                     total_query_rows, scale_log2, causal, num_heads, g.num_kv_heads,
                     g.num_blocks, g.block_stride, g.head_stride, q_tiles);
  return hipGetLastError();
}

template <typename T, int D, int BS>
hipError_t dispatch_group(int group, void* out, const void* query, const void* key_cache,
                          const void* value_cache, const uint32_t* block_tables,
                          int32_t block_table_stride, const uint32_t* cu_seqlens_q,
                          const uint32_t* context_lens, int32_t num_seqs, int32_t max_query_len,
                          int32_t max_kv_len, int64_t total_query_rows, float scale,
                          int32_t causal, int32_t num_heads, const CacheGeom& g,
                          hipStream_t stream) {
#define VPA_PREFILL_G(GG)                                                                       \
  case GG:                                                                                      \
    return launch_prefill_t<T, D, BS, GG>(out, query, key_cache, value_cache, block_tables,    \
                                          block_table_stride, cu_seqlens_q, context_lens,     \
                                          num_seqs, max_query_len, max_kv_len,                 \
                                          total_query_rows, scale, causal, num_heads, g, stream);
  switch (group) {
    VPA_PREFILL_G(1)
    VPA_PREFILL_G(2)
    VPA_PREFILL_G(4)
    default:
      return hipErrorInvalidValue;
  }
#undef VPA_PREFILL_G
}

template <typename T, int D>
hipError_t dispatch_bs(int group, void* out, const void* query, const void* key_cache,
                       const void* value_cache, const uint32_t* block_tables,
                       int32_t block_table_stride, const uint32_t* cu_seqlens_q,
                       const uint32_t* context_lens, int32_t num_seqs, int32_t max_query_len,
                       int32_t max_kv_len, int64_t total_query_rows, float scale, int32_t causal,
                       int32_t num_heads, const CacheGeom& g, hipStream_t stream) {
#define VPA_PREFILL_BS(B)                                                                      \
  case B:                                                                                      \
    return dispatch_group<T, D, B>(group, out, query, key_cache, value_cache, block_tables,   \
                                   block_table_stride, cu_seqlens_q, context_lens, num_seqs, \
                                   max_query_len, max_kv_len, total_query_rows, scale, causal,\
                                   num_heads, g, stream);
  switch (g.block_size) {
    VPA_PREFILL_BS(8)
    VPA_PREFILL_BS(16)
    VPA_PREFILL_BS(32)
    default:
      return hipErrorInvalidValue;
  }
#undef VPA_PREFILL_BS
}

template <typename T>
hipError_t dispatch_dim(int group, void* out, const void* query, const void* key_cache,
                        const void* value_cache, const uint32_t* block_tables,
                        int32_t block_table_stride, const uint32_t* cu_seqlens_q,
                        const uint32_t* context_lens, int32_t num_seqs, int32_t max_query_len,
                        int32_t max_kv_len, int64_t total_query_rows, float scale, int32_t causal,
                        int32_t num_heads, const CacheGeom& g, hipStream_t stream) {
  switch (g.head_dim) {
    case 64:
      return dispatch_bs<T, 64>(group, out, query, key_cache, value_cache, block_tables,
                                block_table_stride, cu_seqlens_q, context_lens, num_seqs,
                                max_query_len, max_kv_len, total_query_rows, scale, causal,
                                num_heads, g, stream);
    case 128:
      return dispatch_bs<T, 128>(group, out, query, key_cache, value_cache, block_tables,
                                 block_table_stride, cu_seqlens_q, context_lens, num_seqs,
                                 max_query_len, max_kv_len, total_query_rows, scale, causal,
                                 num_heads, g, stream);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace

bool prefill_supported(int dtype, int head_dim, int block_size, int group) {
  return (dtype == VPA_DTYPE_BF16 || dtype == VPA_DTYPE_F16) &&
         (head_dim == 64 || head_dim == 128) &&
         (block_size == 8 || block_size == 16 || block_size == 32) &&
         (group == 1 || group == 2 || group == 4);
}

int prefill_positions_per_workgroup(int group) { return 4 * 32 * kPrefillColGroups / group; }

hipError_t launch_prefill_paged(int dtype, void* out, const void* query, const void* key_cache,
                                const void* value_cache, const uint32_t* block_tables,
                                int32_t block_table_stride, const uint32_t* cu_seqlens_q,
                                const uint32_t* context_lens, int32_t num_seqs,
                                int32_t max_query_len, int32_t max_kv_len,
                                int64_t total_query_rows, float scale, int32_t causal,
                                int32_t num_heads, const CacheGeom& g, hipStream_t stream) {
  const int group = num_heads / g.num_kv_heads;
  if (dtype == VPA_DTYPE_BF16)
    return dispatch_dim<bf16_t>(group, out, query, key_cache, value_cache, block_tables,
                                block_table_stride, cu_seqlens_q, context_lens, num_seqs,
                                max_query_len, max_kv_len, total_query_rows, scale, causal,
                                num_heads, g, stream);
  if (dtype == VPA_DTYPE_F16)
    return dispatch_dim<f16_t>(group, out, query, key_cache, value_cache, block_tables,
                               block_table_stride, cu_seqlens_q, context_lens, num_seqs,
                               max_query_len, max_kv_len, total_query_rows, scale, causal,
                               num_heads, g, stream);
  return hipErrorInvalidValue;
}

}  // namespace vpa
