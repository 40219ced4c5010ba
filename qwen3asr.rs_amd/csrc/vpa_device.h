// Device-side helpers shared by the gfx950 kernels: element types, 16-byte
// vector access, conversions and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vpa {

// Storage types. bf16 and f16 are handled as raw 16-bit words so that copies
// stay bit-exact; arithmetic converts explicitly.
struct bf16_t {
  uint16_t x;
};
struct f16_t {
  uint16_t x;
};
// One byte of an fp8 (OCP E4M3FN) cache: bias 7, no infinities, S.1111.111
// is NaN, largest finite 448.
struct fp8_t {
  uint8_t x;
};

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
typedef __attribute__((__vector_size__(2 * sizeof(_Float16)))) _Float16 f16x2_t;

template <typename T>
struct ElemTraits;
template <>
struct ElemTraits<float> {
  static constexpr int kBytes = 4;
};
template <>
struct ElemTraits<bf16_t> {
  static constexpr int kBytes = 2;
};
template <>
struct ElemTraits<f16_t> {
  static constexpr int kBytes = 2;
};
template <>
struct ElemTraits<fp8_t> {
  static constexpr int kBytes = 1;
};

// Elements per 16-byte vector: the key-cache pack factor x of the layout.
template <typename T>
constexpr int pack_x() {
  return 16 / ElemTraits<T>::kBytes;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) {
  return __uint_as_float(b << 16);
}

// Round-to-nearest-even f32 -> bf16 (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, h);
  return (float)v;
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 v = (_Float16)f;
  return __builtin_bit_cast(uint16_t, v);
}

// One element of T widened to f32 (exact).
template <typename T>
__device__ __forceinline__ float load_as_f32(const T* p);
template <>
__device__ __forceinline__ float load_as_f32<float>(const float* p) {
  return *p;
}
template <>
__device__ __forceinline__ float load_as_f32<bf16_t>(const bf16_t* p) {
  return bf16_bits_to_f32(p->x);
}
template <>
__device__ __forceinline__ float load_as_f32<f16_t>(const f16_t* p) {
  return f16_bits_to_f32(p->x);
}

// f32 -> E4M3FN byte: round to nearest even, |x| >= 448 and infinities
// saturate to +-448, NaN gives S.1111.111 (the quantising rule of fp8 KV
// caches). Written out bit by bit so it matches the CPU restatement exactly.
__device__ __forceinline__ uint32_t fp8_from_f32(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7fu;
  if (a >= 0x43e00000u) return sign | 0x7eu;
  if (a < 0x3c800000u)  // below 2^-6: multiples of 2^-9, rint rounds half to even
    return sign | (uint32_t)__builtin_rintf(__uint_as_float(a) * 512.0f);
  const uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
  return sign | ((((r >> 23) - 120u) << 3) | ((r >> 20) & 7u));
}

// Two E4M3FN bytes (byte pair `hi` of a word) -> two packed 16-bit values of
// T (bf16 or f16; exact: every E4M3 value is representable), gfx950's
// v_cvt_scalef32_pk_{bf16,f16}_fp8 with scale 1.
template <typename T>
__device__ __forceinline__ uint32_t fp8x2_to_pk(uint32_t w, bool hi);
template <>
__device__ __forceinline__ uint32_t fp8x2_to_pk<bf16_t>(uint32_t w, bool hi) {
  return hi ? __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true))
            : __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
}
template <>
__device__ __forceinline__ uint32_t fp8x2_to_pk<f16_t>(uint32_t w, bool hi) {
  return hi ? __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true))
            : __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false));
}
// Sixteen E4M3FN bytes -> sixteen values of T in two 16-byte vectors
// (lo: bytes 0..7, hi: bytes 8..15).
template <typename T>
__device__ __forceinline__ void fp8x16_to_pk(const uint4& v, uint4& lo, uint4& hi) {
  lo = make_uint4(fp8x2_to_pk<T>(v.x, false), fp8x2_to_pk<T>(v.x, true),
                  fp8x2_to_pk<T>(v.y, false), fp8x2_to_pk<T>(v.y, true));
  hi = make_uint4(fp8x2_to_pk<T>(v.z, false), fp8x2_to_pk<T>(v.z, true),
                  fp8x2_to_pk<T>(v.w, false), fp8x2_to_pk<T>(v.w, true));
}

template <typename T>
__device__ __forceinline__ void store_from_f32(T* p, float v);
template <>
__device__ __forceinline__ void store_from_f32<float>(float* p, float v) {
  *p = v;
}
template <>
__device__ __forceinline__ void store_from_f32<bf16_t>(bf16_t* p, float v) {
  p->x = f32_to_bf16_bits(v);
}
template <>
__device__ __forceinline__ void store_from_f32<f16_t>(f16_t* p, float v) {
  p->x = f32_to_f16_bits(v);
}

// Two adjacent f32 values packed into one 32-bit word of two 16-bit elements
// (low half = first element).
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi);
template <>
__device__ __forceinline__ uint32_t pack2<bf16_t>(float lo, float hi) {
  return (uint32_t)f32_to_bf16_bits(lo) | ((uint32_t)f32_to_bf16_bits(hi) << 16);
}
template <>
__device__ __forceinline__ uint32_t pack2<f16_t>(float lo, float hi) {
  return (uint32_t)f32_to_f16_bits(lo) | ((uint32_t)f32_to_f16_bits(hi) << 16);
}

// The same packing with gfx950's v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32
// (round to nearest even, one instruction, no branches; a NaN comes out as
// the canonical quiet NaN).
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2v_t __attribute__((ext_vector_type(2)));
template <typename T>
__device__ __forceinline__ uint32_t pack2_hw(float lo, float hi);
template <>
__device__ __forceinline__ uint32_t pack2_hw<bf16_t>(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2v_t));
}
template <>
__device__ __forceinline__ uint32_t pack2_hw<f16_t>(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, f16x2v_t));
}

// acc + a.lo*b.lo + a.hi*b.hi for two packed 16-bit pairs (v_dot2 on gfx950).
template <typename T>
__device__ __forceinline__ float dot2_acc(uint32_t a, uint32_t b, float acc);
template <>
__device__ __forceinline__ float dot2_acc<bf16_t>(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), acc, false);
}
template <>
__device__ __forceinline__ float dot2_acc<f16_t>(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b),
                                acc, false);
}

// Dot product of two 16-byte vectors of T, accumulated in f32.
template <typename T>
__device__ __forceinline__ float dot16(const uint4& a, const uint4& b, float acc) {
  acc = dot2_acc<T>(a.x, b.x, acc);
  acc = dot2_acc<T>(a.y, b.y, acc);
  acc = dot2_acc<T>(a.z, b.z, acc);
  acc = dot2_acc<T>(a.w, b.w, acc);
  return acc;
}
template <>
__device__ __forceinline__ float dot16<float>(const uint4& a, const uint4& b, float acc) {
  acc = fmaf(__uint_as_float(a.x), __uint_as_float(b.x), acc);
  acc = fmaf(__uint_as_float(a.y), __uint_as_float(b.y), acc);
  acc = fmaf(__uint_as_float(a.z), __uint_as_float(b.z), acc);
  acc = fmaf(__uint_as_float(a.w), __uint_as_float(b.w), acc);
  return acc;
}

// Wave64 butterfly reductions; every lane ends with the result.
template <int kFirst, int kLast>
__device__ __forceinline__ float wave_max_range(float v) {
#pragma unroll
  for (int m = kFirst; m <= kLast; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}
template <int kFirst, int kLast>
__device__ __forceinline__ float wave_sum_range(float v) {
#pragma unroll
  for (int m = kFirst; m <= kLast; m <<= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// DPP lane permutations within rows of 16 lanes (gfx9 dpp_ctrl encodings).
template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), kCtrl, 0xf, 0xf, false));
}
constexpr int kDppQuadXor1 = 0xb1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4e;     // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

constexpr int kDppRowRor8 = 0x128;     // lane i <- lane (i + 8) % 16 = i ^ 8 within a row

// v + (v of lane ^ 16) and v + (v of lane ^ 32) with the gfx950 permlane
// swaps (VALU only): swapping a value with itself exchanges rows 0<->1 and
// 2<->3 (16) or the two 32-lane halves (32), and the two results summed
// give the pairwise sum in every lane.
__device__ __forceinline__ float sum_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum over the 64 / BS lanes {l, l ^ BS, ...} that share lane % BS.
template <int BS>
__device__ __forceinline__ float sum_lanes_mod(float v) {
  if constexpr (BS <= 8) v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(
                                                            __builtin_bit_cast(int, v), kDppRowRor8,
                                                            0xf, 0xf, false));
  if constexpr (BS <= 16) v = sum_xor16(v);
  if constexpr (BS <= 32) v = sum_xor32(v);
  return v;
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Full-wave max / sum with DPP inside each 16-lane row and readlane across
// the four rows: no LDS round trips. The result is wave-uniform.
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp<kDppQuadXor1>(v));
  v = fmaxf(v, dpp<kDppQuadXor2>(v));
  v = fmaxf(v, dpp<kDppRowHalfMirror>(v));
  v = fmaxf(v, dpp<kDppRowMirror>(v));
  return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)),
               fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp<kDppQuadXor1>(v);
  v += dpp<kDppQuadXor2>(v);
  v += dpp<kDppRowHalfMirror>(v);
  v += dpp<kDppRowMirror>(v);
  return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}

// Wait until this wave's LDS operations have completed (lgkmcnt(0) only, so
// outstanding global loads stay in flight), and keep the compiler from
// moving LDS accesses across the wait.
__device__ __forceinline__ void lds_wave_sync() {
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
}

// 16-byte load of streamed data (read once): the non-temporal form, which
// keeps it from displacing cached lines (measured on MI355X: a flat
// streaming read reaches 6.96 TB/s with it, 6.23 TB/s with plain loads).
__device__ __forceinline__ uint4 load_stream(const uint4* p) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

}  // namespace vpa
