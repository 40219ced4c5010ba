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
//
// Tile pipeline: the online softmax works on groups of two tiles (one max
// exchange and one rescale test per 64 keys); a pipeline step (one barrier,
// one refill of the other stage buffer) is two tiles for 16-bit caches and
// four for fp8 up to head_dim 128, whose tiles are half the bytes, so two
// steps of four still leave room for two workgroups per CU. Both cache types use the same
// softmax groups, so their rescale points, and with scales 1 their
// results, agree.
// K and V tiles travel HBM -> LDS by the LDS-DMA form of the 16-byte global
// load (no VGPR round trip) into two stage buffers; step t + 1 is issued
// while step t is consumed, waits are explicit vmcnt counts plus a bare
// workgroup barrier (the compiler's __syncthreads would drain every
// outstanding DMA), the block ids of a step are loaded two steps before
// its tiles are consumed, and the operand reads from LDS are
// written as ds_read with their own lgkmcnt wait so the
// compiler does not add a full vmcnt drain before them. Each DMA copies 64
// units of one cache block, so its address is a scalar block base plus a
// fixed per-lane offset. In LDS, K keeps the block's [chunk][key] order and
// V is transposed to [8-key unit][dim]; with the tile's keys permuted inside
// every 16 (tile_key_of_row), each MFMA operand is one 16-byte LDS read and
// every 16-lane read pass covers 256 contiguous bytes (no bank conflicts on
// gfx950's 64 four-byte banks).
//
// Softmax: scores are in log2 units (scale * log2 e folded into the scale);
// the running max only moves when a step's max exceeds it by more than
// kRescaleSlack, so O and the row sums are rescaled rarely and the
// probabilities stay below 2^kRescaleSlack; the result is the same
// sum(p v) / sum(p) for any choice of the reference max.
#include <type_traits>

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

#ifndef VPA_PREFILL_WAVES_PER_EU
#define VPA_PREFILL_WAVES_PER_EU 2
#endif
constexpr int kPrefillKeys = 32;                    // keys per tile
constexpr int kSoftmaxTiles = 2;  // tiles per online-softmax group
// tiles per pipeline step: four for fp8 caches up to head_dim 128 with
// blocks of 16 or 32 tokens (more block ids and DMA offsets per step would
// not fit the scalar registers of the larger shapes), two otherwise
template <bool kF8, int D, int BS>
constexpr int prefill_step_tiles() {
  return kF8 && D <= 128 && BS >= 16 ? 4 : 2;
}
#ifndef VPA_PREFILL_WAVES
#define VPA_PREFILL_WAVES 4
#endif
constexpr int kPrefillWaves = VPA_PREFILL_WAVES;  // waves per workgroup, 32 query rows each
constexpr int kPrefillThreads = 64 * kPrefillWaves;

// s_waitcnt vmcnt(N), leaving the other counters alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// One 16-byte global -> LDS copy per lane (global_load_lds_dwordx4): lane l's
// vector lands at lds + 16 * l; the LDS base is wave-uniform.
__device__ __forceinline__ void dma16(const void* src, const void* lds) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                   (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

template <int N>
using Int = std::integral_constant<int, N>;

typedef int v4i_t __attribute__((ext_vector_type(4)));

// LDS byte address of a __shared__ pointer.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// LDS reads of MFMA operands as inline asm. The tiles arrive by DMA, whose
// completion the kernel waits for explicitly (vmcnt + barrier); reads the
// compiler sees as ordinary LDS loads would get a conservative wait for
// every DMA still in flight, later tiles included. The caller issues an
// s_waitcnt lgkmcnt(0) that names the results before using them.
template <int OFF>
__device__ __forceinline__ v4i_t lds_read_b128(uint32_t addr) {
  v4i_t r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}

typedef int v2i_t __attribute__((ext_vector_type(2)));
template <int OFF>
__device__ __forceinline__ v2i_t lds_read_b64(uint32_t addr) {
  v2i_t r;
  asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
template <int STRIDE, int... I>
__device__ __forceinline__ void lds_read_seq8(v2i_t* dst, uint32_t addr,
                                              std::integer_sequence<int, I...>) {
  ((dst[I] = lds_read_b64<I * STRIDE>(addr)), ...);
}
template <int STRIDE, int SECOND, int... I>
__device__ __forceinline__ void lds_read_pairs8(v2i_t (*dst)[2], uint32_t addr,
                                                std::integer_sequence<int, I...>) {
  ((dst[I][0] = lds_read_b64<I * STRIDE>(addr),
    dst[I][1] = lds_read_b64<I * STRIDE + SECOND>(addr)),
   ...);
}
// Eight E4M3FN bytes -> eight values of T (exact), as one MFMA operand.
template <typename T>
__device__ __forceinline__ v4i_t fp8x8_operand(const v2i_t& b) {
  const uint32_t lo = (uint32_t)b[0], hi = (uint32_t)b[1];
  return v4i_t{(int)fp8x2_to_pk<T>(lo, false), (int)fp8x2_to_pk<T>(lo, true),
               (int)fp8x2_to_pk<T>(hi, false), (int)fp8x2_to_pk<T>(hi, true)};
}

// dst[i] = 16 bytes at addr + i * STRIDE (+ SECOND for dst2), i < N
template <int STRIDE, int... I>
__device__ __forceinline__ void lds_read_seq(v4i_t* dst, uint32_t addr,
                                             std::integer_sequence<int, I...>) {
  ((dst[I] = lds_read_b128<I * STRIDE>(addr)), ...);
}
template <int STRIDE, int SECOND, int... I>
__device__ __forceinline__ void lds_read_pairs(v4i_t (*dst)[2], uint32_t addr,
                                               std::integer_sequence<int, I...>) {
  ((dst[I][0] = lds_read_b128<I * STRIDE>(addr),
    dst[I][1] = lds_read_b128<I * STRIDE + SECOND>(addr)),
   ...);
}

// S^T = K . Q^T of one tile: KS chained MFMAs over the head dimension
template <typename T, int KS>
__device__ __forceinline__ f32x16_t s_tile_mfma(const v4i_t* kop, const uint4* qop) {
  f32x16_t acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const v4i_t k = kop[ks];
    acc = mfma32x32x16<T>(make_uint4(k[0], k[1], k[2], k[3]), qop[ks], acc);
  }
  return acc;
}

// Key held in row i of the S^T tile: bits 2 and 3 of i swapped. Lane half h
// of the 32x32 accumulator holds rows {4h..4h+3, 8+4h..8+4h+3} of every 16;
// through this order those rows are keys 8h..8h+7, one whole 16-byte unit of
// a value row, so the P^T operand of a k-step pairs with one aligned V read.
__device__ __forceinline__ constexpr int tile_key_of_row(int i) {
  return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1);
}

// s_waitcnt lgkmcnt(0) that every one of the M registers just read from LDS
// (by the inline ds_read above) depends on: each is an in-out operand of the
// wait, so no use of it, a register copy included, can be placed before the
// wait. M is 4, 6, 8, 12 or 16 (KS or 2 DT operands at head dims 64 to 256).
template <typename V, int M>
__device__ __forceinline__ void lgkm_wait_flat(V* r) {
  static_assert(M == 4 || M == 6 || M == 8 || M == 12 || M == 16, "operand count");
  if constexpr (M == 4) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]));
  } else if constexpr (M == 6) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]),
                   "+v"(r[4]), "+v"(r[5]));
  } else if constexpr (M == 8) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]),
                   "+v"(r[4]), "+v"(r[5]), "+v"(r[6]), "+v"(r[7]));
  } else if constexpr (M == 12) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]),
                   "+v"(r[4]), "+v"(r[5]), "+v"(r[6]), "+v"(r[7]),
                   "+v"(r[8]), "+v"(r[9]), "+v"(r[10]), "+v"(r[11]));
  } else {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]),
                   "+v"(r[4]), "+v"(r[5]), "+v"(r[6]), "+v"(r[7]),
                   "+v"(r[8]), "+v"(r[9]), "+v"(r[10]), "+v"(r[11]),
                   "+v"(r[12]), "+v"(r[13]), "+v"(r[14]), "+v"(r[15]));
  }
}
template <typename V, int N>
__device__ __forceinline__ void lgkm_wait(V (&r)[N]) {
  lgkm_wait_flat<V, N>(r);
}
template <typename V, int N>
__device__ __forceinline__ void lgkm_wait(V (&r)[N][2]) {
  lgkm_wait_flat<V, 2 * N>(&r[0][0]);
}

// Waves per SIMD the kernel is built for: two up to head_dim 128; above,
// the accumulators and operands of a 32-row wave (O alone is D / 2 VGPRs)
// need the whole register file of one wave.
template <int D>
constexpr int prefill_waves_per_eu() {
  return D > 128 ? 1 : VPA_PREFILL_WAVES_PER_EU;
}

template <typename T, typename C, int D, int BS, int G>
__global__ __launch_bounds__(kPrefillThreads)
__attribute__((amdgpu_waves_per_eu(prefill_waves_per_eu<D>()))) void prefill_paged_kernel(
    T* __restrict__ out, const T* __restrict__ query, const C* __restrict__ key_cache,
    const C* __restrict__ value_cache, const uint32_t* __restrict__ block_tables,
    int32_t block_table_stride, const uint32_t* __restrict__ cu_seqlens_q,
    const uint32_t* __restrict__ context_lens, int32_t num_seqs, int32_t max_query_len,
    int32_t max_kv_len, int64_t total_query_rows, float scale_log2, float denom_eps,
    int32_t causal, int32_t num_heads, int32_t num_kv_heads, int64_t num_blocks,
    int64_t block_stride, int64_t head_stride, int32_t q_tiles, const float* __restrict__ k_scale,
    const float* __restrict__ v_scale) {
  constexpr bool kF8 = std::is_same_v<C, fp8_t>;
  static_assert(kF8 || std::is_same_v<C, T>, "cache type is the query type or fp8");
  constexpr int KT = kPrefillKeys;
  constexpr int SUB = prefill_step_tiles<kF8, D, BS>();
  static_assert(SUB % kSoftmaxTiles == 0, "whole softmax groups per step");
  constexpr int X = kF8 ? 16 : 8;  // cache elements per 16-byte unit
  constexpr int PPW = 32 / G;   // query positions per wave
  constexpr int PPB = kPrefillWaves * PPW;  // query positions per workgroup
  constexpr int KS = D / 16;    // k-steps of Q.K^T
  constexpr int DT = D / 32;    // 32-row tiles of O^T
  // fp8 at 8-token blocks: a 16-byte value unit holds two dims (2r, 2r + 1)
  // of the block's 8 keys and is copied to LDS as it is; otherwise the
  // units of a block's value rows are transposed to [key unit][dim]
  constexpr bool kPairRows = kF8 && BS == 8;
  constexpr int UB = kPairRows ? 1 : BS / X;  // 16-byte units per value row of a block
  constexpr int NU = D * KT / X;                   // 16-byte units per K (and per V) tile
  constexpr int NDMA = NU / 64;                    // DMAs per K (and per V) tile
  // DMAs per issuing wave per K (and per V) tile; the first DMW waves issue
  constexpr int DPW = (NDMA + kPrefillWaves - 1) / kPrefillWaves;
  constexpr int DMW = NDMA / DPW;
  constexpr int NBT = KT / BS;                     // blocks per tile
  constexpr int RBV = D * BS / X;                  // units of one block's K (or V) rows
  constexpr int DPB = RBV / 64;                    // DMAs per block region
  // LDS units between the K regions of two blocks: with 8-key blocks, the 16
  // lanes of one LDS read pass span two blocks, padded to other banks
  constexpr int RBK = RBV + (BS == 8 ? 8 : 0);
  constexpr int KU = NBT * RBK;                    // K units of a stage
  static_assert(KT % BS == 0 && BS >= 8 && NU % 64 == 0 && DMW * DPW == NDMA &&
                    DMW <= kPrefillWaves && RBV % 64 == 0 && (DMW * DPW) % DPB == 0,
                "tile shape");

  // one LDS object per stage: the compiler then knows that a DMA into one
  // stage does not alias the operand reads of another.
  // stage buffer: SUB tiles, each K regions [block][chunk][key], then V
  // regions [block][unit][dim]
  constexpr int TU = KU + NU;  // units of one tile in a stage
  __shared__ __align__(16) uint4 s_t0[SUB * TU], s_t1[SUB * TU];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar branches
  // consecutive workgroups: kv heads, then the query tiles of one sequence
  // (heaviest first), so the tiles of a (sequence, kv head) run together on
  // one XCD and share its K/V through L2
  const int j = (int)(blockIdx.x % (uint32_t)num_kv_heads);
  const int rest = (int)(blockIdx.x / (uint32_t)num_kv_heads);
  const int s = rest / q_tiles;
  const int qt = q_tiles - 1 - rest % q_tiles;

  // The block ids of the first two steps are the first 2 NB0 entries of the
  // table row: loaded here, alongside the sequence's lengths, not after them
  // (up to 4 ids per step: more would not fit the scalar registers of the
  // larger shapes)
  constexpr int NB0 = prefill_step_tiles<kF8, D, BS>() * (kPrefillKeys / BS);
  constexpr bool kEarly = NB0 <= 4;
  const bool early_ids = kEarly && block_table_stride >= 2 * NB0;
  uint32_t w01[kEarly ? 2 * NB0 : 1];
  if (early_ids) {
    const uint32_t* row0 = block_tables + (int64_t)s * block_table_stride;
#pragma unroll
    for (int i = 0; i < 2 * NB0; ++i) w01[i] = row0[i];
  }
  const uint32_t qa = cu_seqlens_q[s], qb = cu_seqlens_q[s + 1];
  const uint32_t ctx = context_lens[s];
  // (all of them in flight together: a load the compiler would sink to its
  // first use, past the early exit, would wait on its own)
  asm volatile("" ::"s"(qa), "s"(qb), "s"(ctx));
  int q_len = qb > qa ? (int)min(qb - qa, (uint32_t)max_query_len) : 0;
  if ((int64_t)qa >= total_query_rows) q_len = 0;
  else q_len = (int)min((int64_t)q_len, total_query_rows - (int64_t)qa);
  const int k_len = (int)min(ctx, (uint32_t)max_kv_len);

  const int p0 = qt * PPB;
  if (p0 >= q_len) return;  // whole workgroup: tile past this sequence's queries
  const int shift = k_len - q_len;  // bottom-right causal alignment
  const int wg_end = min(p0 + PPB, q_len);
  const int n_keys = max(0, causal ? min(k_len, wg_end + shift) : k_len);
  const int n_tiles = (n_keys + KT - 1) / KT;
  const int n_steps = (n_tiles + SUB - 1) / SUB;

  // this lane's query row (column of S^T and O^T)
  const int col = lane & 31;
  const int half = lane >> 5;
  const int wpos0 = p0 + wave * PPW;
  const int pos = wpos0 + col % PPW;
  const int head = j * G + col / PPW;
  const bool row_ok = pos < q_len;
  const int64_t row = (int64_t)qa + pos;
  const int limit = causal ? pos + shift : k_len - 1;  // last key the row sees
  const int wave_end = min(wpos0 + PPW, q_len);
  const int wave_keys =
      wave_end <= wpos0 ? 0 : max(0, causal ? min(k_len, wave_end + shift) : k_len);
  const int wave_min_limit = causal ? wpos0 + shift : k_len - 1;

  // fp8: k_scale folds into the softmax scale (its sign too), v_scale into
  // the output
  float vs = 1.f;
  if constexpr (kF8) {
    scale_log2 *= *k_scale;
    vs = *v_scale;
  }
  uint4 qop[KS];
  {
    // (every lane loads: a row past the sequence's queries reads its first
    // row instead, in bounds, so the loads need no branch; such a row's
    // scores and output stay in its own lane and column and are not stored)
    const T* qrow = query + ((row_ok ? row : (int64_t)qa) * num_heads + head) * D + 8 * half;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qop[ks] = *reinterpret_cast<const uint4*>(qrow + 16 * ks);
    // a negative scale is folded into Q (a sign flip, exact in the cache
    // type), so the row max can be taken on the raw scores
    if (scale_log2 < 0.f) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        qop[ks].x ^= 0x80008000u;
        qop[ks].y ^= 0x80008000u;
        qop[ks].z ^= 0x80008000u;
        qop[ks].w ^= 0x80008000u;
      }
    }
  }

  f32x16_t o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.f;
  const float sl = fabsf(scale_log2);
  float m = -INFINITY;   // reference max of the row (moves lazily), log2 units
  float mt = -INFINITY;  // the row's true max so far, log2 units
  float lsum = 0.f;      // this lane's share of the row's exp sum

  const C* kbase = key_cache + (int64_t)j * head_stride;
  const C* vbase = value_cache + (int64_t)j * head_stride;
  const uint32_t* bt = block_tables + (int64_t)s * block_table_stride;
  const char* kbytes = reinterpret_cast<const char*>(kbase);
  const char* vbytes = reinterpret_cast<const char*>(vbase);
  const uint64_t bstride_b = (uint64_t)block_stride * sizeof(C);  // bytes between blocks
  const int last_blk = max(k_len - 1, 0) / BS;
  // every u32 block id is inside the pool (the id checks compare 32 bits,
  // in scalar registers, otherwise)
  const bool huge_pool = num_blocks > (int64_t)0xffffffffu;
  // largest block id inside the pool, as 32 bits (one compare per id)
  const uint32_t max_id = huge_pool ? 0xffffffffu : (uint32_t)(num_blocks - 1);

  // K and V regions of tile u of stage S
  auto kst = [&](auto sc, int u) -> uint4* {
    constexpr int S = decltype(sc)::value;
    if constexpr (S == 0) return s_t0 + u * TU;
    else return s_t1 + u * TU;
  };
  auto vst = [&](auto sc, int u) -> uint4* { return kst(sc, u) + KU; };
  // block ids of a tile (uniform: scalar loads; the index is clamped to the
  // sequence's last block, which exists whenever a tile is touched)
  auto tile_blocks = [&](int k0, uint32_t (&pb)[NBT]) {
#pragma unroll
    for (int i = 0; i < NBT; ++i)
      pb[i] = bt[__builtin_amdgcn_readfirstlane(min(k0 / BS + i, last_blk))];
  };
  // Every DMA copies 64 units of one block (DPB DMAs per block region), so
  // its global base is uniform and each lane adds a fixed element offset:
  // K regions are plain copies of the block's [chunk][key] units, V regions
  // transpose the block's [dim][unit] rows to [unit][dim].
  uint32_t koffb[DPW], voffb[DPW];  // bytes
#pragma unroll
  for (int i = 0; i < DPW; ++i) {
    const int r = ((wave * DPW + i) % DPB) * 64 + lane;  // unit of the block region
    koffb[i] = (uint32_t)(r * X) * (uint32_t)sizeof(C);
    voffb[i] = (kPairRows ? (uint32_t)(r * X) : (uint32_t)((r % D) * BS + (r / D) * X)) *
               (uint32_t)sizeof(C);
  }

  // Issue the DMAs of the SUB tiles of step t into stage S (always all SUB
  // of them, so every step moves the same count). Keys past the context and
  // absent blocks read block 0 (in bounds); they are masked in S and their
  // values zeroed when the V operands are built.
  // block ids of the SUB tiles of step t
  // (with a table row of at least NB entries: one NB-dword scalar load of the
  // window of the row that starts at the step's first block, clamped to the
  // sequence's last one. Entries past the last block are whatever the row
  // holds there: their keys are masked and their DMAs read block 0. Only
  // where the row ends inside the window are the entries loaded one by one,
  // clamped to the last block. The load has no branch around it to merge
  // with, so its wait lands at the ids' first use, a step later.)
  constexpr int NB = SUB * NBT;  // block ids of a step
  const bool wide_ids = block_table_stride >= NB;
  auto step_blocks = [&](int t, uint32_t (&pbs)[SUB][NBT]) {
    if (!wide_ids) {
#pragma unroll
      for (int u = 0; u < SUB; ++u) tile_blocks((t * SUB + u) * KT, pbs[u]);
      return;
    }
    const int first = __builtin_amdgcn_readfirstlane(min(t * SUB * KT / BS, last_blk));
    const int base = min(first, block_table_stride - NB);
    uint32_t w[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) w[i] = bt[base + i];
    if (base != first) {  // rare: the table row ends inside the window
#pragma unroll
      for (int i = 0; i < NB; ++i) w[i] = bt[min(first + i, last_blk)];
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) pbs[i / NBT][i % NBT] = w[i];
  };
  // (full: every block of the step inside the pool and every key inside the
  // context, so the ids are used unchecked)
  auto issue = [&](auto sc, auto full, int t, const uint32_t (&pbs)[SUB][NBT]) {
    if (DMW < kPrefillWaves && wave >= DMW) return;  // wave issues no DMA (uniform)
#pragma unroll
    for (int u = 0; u < SUB; ++u) {
      const int k0 = (t * SUB + u) * KT;
      const uint32_t(&pb)[NBT] = pbs[u];
      uint4* sk = kst(sc, u);
      uint4* sv = vst(sc, u);
#pragma unroll
      for (int i = 0; i < DPW; ++i) {
        const int di = wave * DPW + i;  // uniform
        const int b = di / DPB;
        uint32_t phys;
        if constexpr (NBT <= 2) {
          // (select between values, not between array elements: a select
          // of two loads would become one runtime-indexed load and keep the
          // block ids in scratch memory)
          const uint32_t id0 = __builtin_amdgcn_readfirstlane(pb[0]);
          const uint32_t id1 = __builtin_amdgcn_readfirstlane(pb[NBT - 1]);
          phys = b == 0 ? id0 : id1;
        } else {
          // (a select over more blocks by the runtime index b becomes an
          // indexed scratch array: load the id from the table instead)
          phys = bt[__builtin_amdgcn_readfirstlane(min(k0 / BS + b, last_blk))];
        }
        if constexpr (!decltype(full)::value)
          phys = (k0 + b * BS < k_len && phys <= max_id) ? phys : 0u;
        phys = __builtin_amdgcn_readfirstlane(phys);
        // the block's byte offset in scalar registers (the compiler would
        // otherwise fuse the multiply into a 64-bit vector multiply-add per
        // DMA)
        const uint64_t blk = (uint64_t)phys * bstride_b;
        const uint64_t ub =
            ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(blk >> 32)) << 32) |
            __builtin_amdgcn_readfirstlane((uint32_t)blk);
        dma16(kbytes + ub + koffb[i], sk + b * RBK + (di % DPB) * 64);
        dma16(vbytes + ub + voffb[i], sv + b * RBV + (di % DPB) * 64);
      }
    }
  };

  // LDS byte offsets of this lane's operand reads within a stage
  // (16-bit: chunk 2 ks + half of the key, one unit; fp8: bytes 8 half ..
  // 8 half + 7 of chunk ks)
  const uint32_t ka_lane = [&] {
    const int key = tile_key_of_row(col);
    if constexpr (kF8) return (uint32_t)(((key / BS) * RBK + key % BS) * 16 + 8 * half);
    else return (uint32_t)(((key / BS) * RBK + half * BS + key % BS) * 16);
  }();
  // unit group g = 2 k2 + half of the tile (keys 8g .. 8g+7) sits at
  // (g / UB) * RBV + (g % UB) * D units; that splits into a k2 and a half term
  // (fp8: units hold 16 keys; keys 8g .. 8g+7 are bytes 8 (g % 2) .. of
  // unit g / 2)
  // (fp8 at 8-token blocks: keys 8g .. 8g+7 of dim d are bytes 8 (d % 2) ..
  // of unit d / 2 of block region g)
  auto vgroup = [](int g) { return (g / UB) * RBV + (g % UB) * D; };
  constexpr int kVStep1 = kPairRows ? 2 * RBV * 16
                          : kF8     ? ((1 / UB) * RBV + (1 % UB) * D) * 16
                                    : ((2 / UB) * RBV + (2 % UB) * D) * 16;
  constexpr int kVStepD = kPairRows ? 32 * 8 : 32 * 16;  // LDS bytes between 32-dim tiles
  const uint32_t va_lane = kPairRows ? (uint32_t)(half * RBV * 16 + col * 8)
                           : kF8     ? (uint32_t)(col * 16 + 8 * half)
                                     : (uint32_t)((vgroup(half) + col) * 16);

  // keys of tile t that exist: inside the context and in a present block
  // (uniform over the workgroup)
  // (present: bit kb set when block kb of the tile is inside the pool)
  auto tile_mask = [&](int t, uint32_t present) {
    const int k0 = t * KT;
    uint32_t vmask = 0;
#pragma unroll
    for (int kb = 0; kb < NBT; ++kb)
      if ((present >> kb) & 1u)
        vmask |= (BS >= 32 ? 0xffffffffu : ((1u << BS) - 1u)) << (kb * BS);
    const int nk = k_len - k0;
    if (nk < KT) vmask &= (1u << max(nk, 0)) - 1u;
    return vmask;
  };

  // Zero the LDS values of the keys vmask leaves out: their slots hold
  // stale data (maybe NaN), and a zero probability times NaN would poison O.
  // Element k % X of unit (k / X, d) holds key k of dim d.
  auto zero_absent_values = [&](uint4* sv, uint32_t vmask) {
    using E = std::conditional_t<kF8, uint8_t, uint16_t>;
    E* ve = reinterpret_cast<E*>(sv);
    const uint32_t absent = ~vmask;
    for (int e = tid; e < KT * D; e += kPrefillThreads) {
      const int k = e / D, d = e % D;
      if ((absent >> k) & 1u) {
        if constexpr (kPairRows) ve[(k / BS) * RBV * 16 + d * 8 + k % BS] = 0;
        else ve[(vgroup(k / X) + d) * X + k % X] = 0;
      }
    }
  };

  // S^T of one tile (keys k0 .. k0 + 31) with the keys this lane's row does
  // not see at -inf
  auto scores = [&](const uint4* sk, int k0, uint32_t vmask) -> f32x16_t {
    const bool full = vmask == 0xffffffffu && k0 + KT - 1 <= wave_min_limit;

    // S^T = K . Q^T; the K operand of k-step ks is chunk 2 ks + half of the
    // key in row col
    v4i_t kop[KS];
    if constexpr (kF8) {
      v2i_t k8[KS];
      lds_read_seq8<BS * 16>(k8, ka_lane + lds_addr(sk), std::make_integer_sequence<int, KS>{});
      lgkm_wait(k8);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kop[ks] = fp8x8_operand<T>(k8[ks]);
    } else {
      lds_read_seq<2 * BS * 16>(kop, ka_lane + lds_addr(sk),
                                std::make_integer_sequence<int, KS>{});
      lgkm_wait(kop);
    }
    f32x16_t sacc = s_tile_mfma<T, KS>(kop, qop);
    if (!full) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = 16 * (r / 8) + 8 * half + r % 8;  // key of element r
        const bool ok = ((vmask >> key) & 1u) && k0 + key <= limit;
        sacc[r] = ok ? sacc[r] : -INFINITY;
      }
    }
    return sacc;
  };

  // probabilities of one tile against the reference max, added to the row
  // sum; O^T += V^T . P^T with P^T straight from the accumulator
  auto accumulate = [&](const uint4* sv, const f32x16_t& sacc, float m_use) {
    float sval[16];
#pragma unroll
    for (int r = 0; r < 16; ++r)
      sval[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[r], sl, -m_use));
    float ps = sval[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) ps += sval[r];
    lsum += ps;
    uint4 pk[2];
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2)
      pk[k2] = make_uint4(pack2_hw<T>(sval[8 * k2 + 0], sval[8 * k2 + 1]),
                          pack2_hw<T>(sval[8 * k2 + 2], sval[8 * k2 + 3]),
                          pack2_hw<T>(sval[8 * k2 + 4], sval[8 * k2 + 5]),
                          pack2_hw<T>(sval[8 * k2 + 6], sval[8 * k2 + 7]));
    // k-step k2 of lane half h covers keys 16 k2 + 8h .. 16 k2 + 8h + 7, one
    // unit of row d = 32 dt + col (values of absent keys were zeroed in LDS
    // by the step)
    v4i_t vop[DT][2];
    if constexpr (kF8) {
      v2i_t v8[DT][2];
      lds_read_pairs8<kVStepD, kVStep1>(v8, va_lane + lds_addr(sv),
                                        std::make_integer_sequence<int, DT>{});
      lgkm_wait(v8);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) vop[dt][k2] = fp8x8_operand<T>(v8[dt][k2]);
    } else {
      lds_read_pairs<32 * 16, kVStep1>(vop, va_lane + lds_addr(sv),
                                       std::make_integer_sequence<int, DT>{});
      lgkm_wait(vop);
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2)
        o[dt] = mfma32x32x16<T>(__builtin_bit_cast(uint4, vop[dt][k2]), pk[k2], o[dt]);
  };

  // the SUB tiles of step t in softmax groups of two: scores of both tiles
  // of a group, one online-softmax update for the group (on the raw scores;
  // the scale is positive), then P.V of each
  auto compute = [&](auto sc, int t, const uint32_t (&vmask)[SUB]) {
#pragma unroll
    for (int g0 = 0; g0 < SUB; g0 += kSoftmaxTiles) {
      const int k0 = (t * SUB + g0) * KT;
      if (k0 >= wave_keys) return;  // no row of this wave sees these keys
      // (every tile of the group is scored: one past this wave's keys is
      // masked whole, which is cheaper than the -inf fill the compiler would
      // otherwise hoist into the common path)
      f32x16_t sacc[kSoftmaxTiles];
#pragma unroll
      for (int u = 0; u < kSoftmaxTiles; ++u)
        sacc[u] = scores(kst(sc, g0 + u), k0 + u * KT, vmask[g0 + u]);
      float mx = -INFINITY;
#pragma unroll
      for (int u = 0; u < kSoftmaxTiles; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[u][r]);
      mx = max_xor32(mx) * sl;
      mt = fmaxf(mt, mx);
      // The reference max m only moves when some row's group max exceeds it
      // by more than kRescaleSlack (log2 units): the probabilities stay below
      // 2^kRescaleSlack, and O and the row sums are rescaled only then.
      constexpr float kRescaleSlack = 8.f;
      if (__ballot(mx > m + kRescaleSlack) != 0) {
        const float m_new = fmaxf(m, mx);
        const float alpha = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - m_new);
        lsum *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int e = 0; e < 16; ++e) o[dt][e] *= alpha;
        m = m_new;
      }
      const float m_use = m == -INFINITY ? 0.f : m;  // a row without keys so far
      accumulate(vst(sc, g0), sacc[0], m_use);
#pragma unroll
      for (int u = 1; u < kSoftmaxTiles; ++u)
        if (k0 + u * KT < wave_keys) accumulate(vst(sc, g0 + u), sacc[u], m_use);
    }
  };

  // bit u NBT + kb: block kb of tile u of a step is inside the pool
  auto step_present = [&](const uint32_t (&pbs)[SUB][NBT]) {
    uint32_t bits = 0;
#pragma unroll
    for (int u = 0; u < SUB; ++u)
#pragma unroll
      for (int kb = 0; kb < NBT; ++kb)
        bits |= (pbs[u][kb] <= max_id ? 1u : 0u) << (u * NBT + kb);
    return bits;
  };
  static_assert(SUB * NBT <= 32, "presence bits of a step");

  // one pipeline step: wait for step t's tiles, refill the stage step t-1
  // used with step t + 1, compute step t. The block ids travel ahead of the
  // steps: pi (step t + 1, for the DMAs issued here) was loaded one step
  // earlier and the ids of step t + 2 are loaded into pf here, so no step
  // waits for a table load; the masks of step t need only which of its
  // blocks are inside the pool (pres, worked out when its DMAs were issued,
  // as "all of them" or 0 for "work the bits out"; pres_next gets step
  // t + 1's).
  // (With four blocks per tile the DMAs load their block ids from the table
  // themselves and the registers of two steps' ids would not fit the larger
  // shapes: each step then loads its own ids, before its waits, for the
  // masks, and pi / pf are not used.)
  constexpr bool kCarryIds = NBT <= 2;
  auto step = [&](auto sc, int t, uint32_t pres, const uint32_t (&pi)[SUB][NBT],
                  uint32_t (&pf)[SUB][NBT], uint32_t& pres_next) {
    if (t >= n_steps) return;
    constexpr int S = decltype(sc)::value;
    const bool refill = t + 1 < n_steps;
    if constexpr (kCarryIds) {
      step_blocks(t + 2, pf);  // (past the last step: loaded, not used)
    } else {
      uint32_t own[SUB][NBT];
      step_blocks(t, own);
      pres = step_present(own);
    }
    wait_vmcnt<0>();  // step t's DMAs (the only ones in flight)
    // step t is in LDS for every wave, and every wave is done with step t-1.
    // A bare s_barrier: __syncthreads() would also fence this wave's LDS
    // writes, i.e. wait for all of its outstanding DMAs; the explicit vmcnt
    // wait above already covers step t.
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    uint32_t vmask[SUB];
    bool fix = false;
    // The common step, every block in the pool and every key in the
    // context, takes full masks without working them out: the scalar
    // instructions of a step sit in each wave's issue stream ahead of its
    // MFMAs (about 30 fewer per step here: 3 % on c4).
    constexpr uint32_t kAllPresent = SUB * NBT >= 32 ? 0xffffffffu : (1u << (SUB * NBT)) - 1u;
    if (pres == kAllPresent && (t + 1) * (SUB * KT) <= k_len) {
#pragma unroll
      for (int u = 0; u < SUB; ++u) vmask[u] = 0xffffffffu;
    } else {
      if constexpr (kCarryIds) {
        if (pres != kAllPresent) {  // some block may be absent: the step's ids again
          uint32_t own[SUB][NBT];
          step_blocks(t, own);
          pres = step_present(own);
        }
      }
#pragma unroll
      for (int u = 0; u < SUB; ++u) {
        vmask[u] = tile_mask(t * SUB + u, (pres >> (u * NBT)) & ((1u << NBT) - 1u));
        // tiles past the last one are read by no wave
        fix |= vmask[u] != 0xffffffffu && t * SUB + u < n_tiles;
      }
    }
    if (fix) {  // rare: the sequence's last tile, absent blocks
#pragma unroll
      for (int u = 0; u < SUB; ++u)
        if (vmask[u] != 0xffffffffu && t * SUB + u < n_tiles)
          zero_absent_values(vst(sc, u), vmask[u]);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    }
    if (refill) {
      if constexpr (kCarryIds) {
        // only whether every block is in the pool is worked out ahead (a
        // maximum over the ids); a step with an absent block reloads its ids
        // for the bits
        uint32_t mx = pi[0][0];
#pragma unroll
        for (int u = 0; u < SUB; ++u)
#pragma unroll
          for (int kb = 0; kb < NBT; ++kb) mx = max(mx, pi[u][kb]);
        pres_next = mx <= max_id ? kAllPresent : 0u;
        if (pres_next == kAllPresent && (t + 2) * (SUB * KT) <= k_len)
          issue(Int<1 - S>{}, std::true_type{}, t + 1, pi);
        else
          issue(Int<1 - S>{}, std::false_type{}, t + 1, pi);
      } else {
        issue(Int<1 - S>{}, std::false_type{}, t + 1, pi);
      }
    }
    compute(sc, t, vmask);
  };
  if (n_steps > 0) {
    // ids of the step whose DMAs come next (x at even steps, y at odd ones)
    // and of the one after it; presence bits of the current and next step
    uint32_t ix[SUB][NBT] = {}, iy[SUB][NBT] = {};
    uint32_t p0 = 0, p1 = 0;
    // ids of step t in {0, 1}: entries t NB0 .. t NB0 + NB0 - 1 of the row
    // (entries past the sequence's last block are never dereferenced: their
    // keys lie past the context, so their DMAs read block 0 and their keys
    // are masked)
    auto early_blocks = [&](int t, uint32_t (&pbs)[SUB][NBT]) {
      if constexpr (kEarly) {
#pragma unroll
        for (int i = 0; i < NB0; ++i) pbs[i / NBT][i % NBT] = w01[t * NB0 + i];
      }
    };
    if (early_ids) early_blocks(0, ix);
    else step_blocks(0, ix);
    p0 = step_present(ix);
    issue(Int<0>{}, std::false_type{}, 0, ix);
    if (kCarryIds && 1 < n_steps) {
      if (early_ids) early_blocks(1, ix);
      else step_blocks(1, ix);
    }
    for (int t0 = 0; t0 < n_steps; t0 += 2) {
      step(Int<0>{}, t0, p0, ix, iy, p1);      // loads the ids of t0 + 2 into iy
      step(Int<1>{}, t0 + 1, p1, iy, ix, p0);  // loads the ids of t0 + 3 into ix
    }
  }

  // the denominator's epsilon is relative to the row's true max: the sums
  // here are relative to m, 2^(mt - m) (at most 2^kRescaleSlack) times
  // larger
  const float total = sum_xor32(lsum);
  const float eps_m = denom_eps > 0.f && m != -INFINITY
                          ? denom_eps * __builtin_amdgcn_exp2f(mt - m)
                          : 0.f;
  const float inv = total > 0.f ? vs / (total + eps_m) : 0.f;  // a row that sees no key gives 0
  if (row_ok) {
    T* orow = out + (row * num_heads + head) * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d0 = 32 * dt + 8 * i + 4 * half;
        *reinterpret_cast<uint2*>(orow + d0) =
            make_uint2(pack2_hw<T>(o[dt][4 * i] * inv, o[dt][4 * i + 1] * inv),
                       pack2_hw<T>(o[dt][4 * i + 2] * inv, o[dt][4 * i + 3] * inv));
      }
  }
}

// Arguments after the template dispatch, shared by every instance.
struct PrefillArgs {
  void* out;
  const void* query;
  const void* key_cache;
  const void* value_cache;
  const uint32_t* block_tables;
  int32_t block_table_stride;
  const uint32_t* cu_seqlens_q;
  const uint32_t* context_lens;
  int32_t num_seqs, max_query_len, max_kv_len;
  int64_t total_query_rows;
  float scale;
  float denom_eps;
  int32_t causal, num_heads;
  const float* k_scale;
  const float* v_scale;
};

template <typename T, typename C, int D, int BS, int G>
hipError_t launch_prefill_t(const PrefillArgs& a, const CacheGeom& g, hipStream_t stream) {
  constexpr int kPositions = kPrefillWaves * 32 / G;
  const int q_tiles = (a.max_query_len + kPositions - 1) / kPositions;
  const int64_t grid = (int64_t)a.num_seqs * q_tiles * g.num_kv_heads;
  if (grid == 0) return hipSuccess;
  const float scale_log2 = a.scale * 1.4426950408889634f;
  hipLaunchKernelGGL((prefill_paged_kernel<T, C, D, BS, G>), dim3((uint32_t)grid),
                     dim3(kPrefillThreads), 0, stream, static_cast<T*>(a.out),
                     static_cast<const T*>(a.query), static_cast<const C*>(a.key_cache),
                     static_cast<const C*>(a.value_cache), a.block_tables, a.block_table_stride,
                     a.cu_seqlens_q, a.context_lens, a.num_seqs, a.max_query_len, a.max_kv_len,
                     a.total_query_rows, scale_log2, a.denom_eps, a.causal, a.num_heads,
                     g.num_kv_heads,
                     g.num_blocks, g.block_stride, g.head_stride, q_tiles, a.k_scale,
                     a.v_scale);
  return hipGetLastError();
}

template <typename T, typename C, int D, int BS>
hipError_t dispatch_group(int group, const PrefillArgs& a, const CacheGeom& g,
                          hipStream_t stream) {
  switch (group) {
    case 1:
      return launch_prefill_t<T, C, D, BS, 1>(a, g, stream);
    case 2:
      return launch_prefill_t<T, C, D, BS, 2>(a, g, stream);
    case 4:
      return launch_prefill_t<T, C, D, BS, 4>(a, g, stream);
    default:
      return hipErrorInvalidValue;
  }
}

// Shapes: head_dim 64, 96, 128, 192 or 256, block sizes 8, 16, 32, with a
// (block, head) tile of a whole number of 1 KiB DMAs (D * BS / x a multiple
// of 64 units): head_dim 96 at 16-bit needs 16- or 32-token blocks, at fp8
// 32-token ones; fp8 at 8-token blocks takes head_dim 128 and 256. At fp8
// head_dim 64 a 32-key tile is 128 units, moved by two of the four waves.
constexpr bool prefill_shape(bool fp8, int d, int bs) {
  const int x = fp8 ? 16 : 8;
  const bool dim = d == 64 || d == 96 || d == 128 || d == 192 || d == 256;
  const bool blk = bs == 8 || bs == 16 || bs == 32;
  return dim && blk && (d * bs / x) % 64 == 0;
}

template <typename T, typename C, int D, int BS>
hipError_t dispatch_if(int group, const PrefillArgs& a, const CacheGeom& g, hipStream_t stream,
                       bool& done) {
  constexpr bool kF8 = std::is_same_v<C, fp8_t>;
  if constexpr (prefill_shape(kF8, D, BS)) {
    if (g.head_dim == D && g.block_size == BS) {
      done = true;
      return dispatch_group<T, C, D, BS>(group, a, g, stream);
    }
  }
  return hipSuccess;
}

template <typename T, typename C, int D>
hipError_t dispatch_dim(int group, const PrefillArgs& a, const CacheGeom& g, hipStream_t stream,
                        bool& done) {
  hipError_t e = dispatch_if<T, C, D, 8>(group, a, g, stream, done);
  if (!done) e = dispatch_if<T, C, D, 16>(group, a, g, stream, done);
  if (!done) e = dispatch_if<T, C, D, 32>(group, a, g, stream, done);
  return e;
}

template <typename T, typename C>
hipError_t dispatch_shape(int group, const PrefillArgs& a, const CacheGeom& g,
                          hipStream_t stream) {
  bool done = false;
  hipError_t e = dispatch_dim<T, C, 128>(group, a, g, stream, done);
  if (!done) e = dispatch_dim<T, C, 64>(group, a, g, stream, done);
  if (!done) e = dispatch_dim<T, C, 96>(group, a, g, stream, done);
  if (!done) e = dispatch_dim<T, C, 192>(group, a, g, stream, done);
  if (!done) e = dispatch_dim<T, C, 256>(group, a, g, stream, done);
  return done ? e : hipErrorInvalidValue;
}

}  // namespace

bool prefill_supported(int dtype, int cache_dtype, int head_dim, int block_size, int group) {
  if (!(dtype == VPA_DTYPE_BF16 || dtype == VPA_DTYPE_F16) || !(group == 1 || group == 2 ||
                                                                group == 4))
    return false;
  const bool fp8 = cache_dtype == VPA_DTYPE_FP8_E4M3;
  if (!fp8 && cache_dtype != dtype) return false;
  return prefill_shape(fp8, head_dim, block_size);
}

int prefill_positions_per_workgroup(int group) { return kPrefillWaves * 32 / group; }

hipError_t launch_prefill_paged(int dtype, int cache_dtype, void* out, const void* query,
                                const void* key_cache, const void* value_cache,
                                const uint32_t* block_tables, int32_t block_table_stride,
                                const uint32_t* cu_seqlens_q, const uint32_t* context_lens,
                                int32_t num_seqs, int32_t max_query_len, int32_t max_kv_len,
                                int64_t total_query_rows, float scale, float denom_eps,
                                int32_t causal, int32_t num_heads, const CacheGeom& g,
                                const float* k_scale, const float* v_scale,
                                hipStream_t stream) {
  const int group = num_heads / g.num_kv_heads;
  const PrefillArgs a{out,       query,        key_cache,      value_cache,  block_tables,
                      block_table_stride,      cu_seqlens_q,   context_lens, num_seqs,
                      max_query_len,           max_kv_len,     total_query_rows,
                      scale,     denom_eps,    causal,         num_heads,    k_scale,
                      v_scale};
  const bool f8 = cache_dtype == VPA_DTYPE_FP8_E4M3;
  if (dtype == VPA_DTYPE_BF16)
    return f8 ? dispatch_shape<bf16_t, fp8_t>(group, a, g, stream)
              : dispatch_shape<bf16_t, bf16_t>(group, a, g, stream);
  if (dtype == VPA_DTYPE_F16)
    return f8 ? dispatch_shape<f16_t, fp8_t>(group, a, g, stream)
              : dispatch_shape<f16_t, f16_t>(group, a, g, stream);
  return hipErrorInvalidValue;
}

}  // namespace vpa
