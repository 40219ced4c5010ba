/*
 * vpa_oracle.c — TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of the reference's paged-KV hot path, used as the checker
 * for the HIP kernels and as the CPU baseline that bench.py times. Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library; the product (libvpa) never calls it.
 *
 * The kernels the reference calls (reshape_and_cache, paged_attention,
 * gather_kv_cache) live in the external crate mistralrs-paged-attn 0.8.3
 * (git gitee.com/good-as-water/mistral.rs rev 0a14af4a, pinned at
 * vasr-paged-attn/Cargo.toml:15 and Cargo.lock:2601-2615), which is not
 * vendored. What is restated here is the semantics the reference's own files
 * fix for them:
 *   - cache layout and its inverse: vasr-paged-attn/src/paged_kv_cache.rs:263-294
 *     and vasr-models/src/model/generation.rs:338-440;
 *   - slot -> (block, offset) and PAD_SLOT_ID = -1 skip:
 *     paged_kv_cache.rs:7, 74-103, 697-700;
 *   - the paged K/V indexing of the in-tree sibling kernel:
 *     vasr-paged-attn/src/metal/kernels/prefill_paged_attn.metal:1203-1214
 *     (K) and :1272-1283 (V), and its 1e-6 denominator term (:1300);
 *   - GQA head map kvh = h / (H / KVH): vasr-models/src/model/attention.rs:12-21;
 *   - eager attention QK^T*scale -> softmax -> .V: attention.rs:243-286;
 *   - cached causal mask, query q at absolute position cache_len + q sees keys
 *     <= that position: attention.rs:78-149;
 *   - contiguous KV append of the CPU path: vasr-models/src/model/kv_cache.rs:54-111.
 *
 * Checker functions accumulate in double. The cpu_baseline_* functions are
 * the reference's CPU path restated in f32 with OpenMP over (seq, kv head)
 * for timing only.
 *
 * Element types: 0 = f32, 1 = f16, 2 = bf16, 3 = fp8 E4M3FN (cache only;
 * same codes as include/vpa.h). 16-bit elements are raw uint16_t words, fp8
 * elements raw bytes.
 *
 * FP8 cache (the reference's uint8 cache variant): decode of a byte follows
 * the E4M3FN format the reference's Metal kernels read
 * (vasr-paged-attn/src/metal/kernels/prefill_paged_attn.metal:698-722), and a
 * cached value is dequantised as (float)byte * scale rounded to the query
 * type (:764-769). The quantising side, reshape_and_cache into an fp8 cache,
 * lives in the un-vendored mistralrs-paged-attn crate; its published rule
 * (the vLLM kernels it derives from) is byte = E4M3FN(x / scale) with
 * round-to-nearest-even and saturation to the largest finite value (448),
 * NaN staying NaN. Both directions are pinned in tests/test_oracle.py
 * against torch.float8_e4m3fn and the format's closed forms.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_F32 0
#define ORC_F16 1
#define ORC_BF16 2
#define ORC_FP8 3

static int elem_bytes(int dtype) { return dtype == ORC_F32 ? 4 : (dtype == ORC_FP8 ? 1 : 2); }

static uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* E4M3FN byte -> binary32, exact: bias 7, no infinities, S.1111.111 = NaN,
 * exponent field 0 = subnormal m * 2^-9. */
float oracle_fp8_to_f32(uint8_t v) {
  const uint32_t sign = (uint32_t)(v & 0x80) << 24;
  const uint32_t e = (v >> 3) & 0xf, m = v & 7;
  if (e == 0xf && m == 7) return bits_f32(sign | 0x7fc00000u);
  if (e == 0) {
    const float mag = (float)m * 0x1p-9f;
    return (v & 0x80) ? -mag : mag;
  }
  return bits_f32(sign | ((e + 120) << 23) | (m << 20));
}

/* binary32 -> E4M3FN byte: round to nearest, ties to even; |x| >= 448 (and
 * infinities) saturate to +-448; NaN gives S.1111.111. */
uint8_t oracle_fp8_from_f32(float x) {
  const uint32_t u = f32_bits(x);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7f;  /* NaN */
  if (a >= 0x43e00000u) return sign | 0x7e; /* >= 448: largest finite */
  if (a < 0x3c800000u) {                    /* below 2^-6: multiples of 2^-9 */
    const float t = bits_f32(a) * 512.0f;   /* exact */
    float r = floorf(t);
    const float frac = t - r;
    if (frac > 0.5f || (frac == 0.5f && fmodf(r, 2.0f) == 1.0f)) r += 1.0f;
    return sign | (uint8_t)r;                /* r == 8 is 2^-6, the first normal */
  }
  const uint32_t lsb = (a >> 20) & 1;
  const uint32_t r = a + 0x7ffffu + lsb;    /* round the 23-bit mantissa to 3 bits */
  const uint32_t e = (r >> 23) - 120, m = (r >> 20) & 7;
  return sign | (uint8_t)((e << 3) | m);
}

void oracle_fp8_to_f32_array(const uint8_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_fp8_to_f32(in[i]);
}
void oracle_fp8_from_f32_array(const float* in, uint8_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_fp8_from_f32(in[i]);
}

/* binary32 -> bf16 / binary16 words, round to nearest even (NaN kept). */
static uint16_t f32_to_bf16_rne(float f) {
  const uint32_t u = f32_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1)) >> 16);
}
static uint16_t f32_to_f16_rne(float f) {
  const uint32_t u = f32_bits(f);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7e00;                   /* NaN */
  if (a >= 0x477ff000u) return sign | 0x7c00;                  /* rounds past 65504: inf */
  if (a < 0x38800000u) {                                       /* below 2^-14: subnormal */
    const double t = (double)bits_f32(a) * 16777216.0;          /* units of 2^-24, exact */
    double r = floor(t);
    const double frac = t - r;
    if (frac > 0.5 || (frac == 0.5 && fmod(r, 2.0) == 1.0)) r += 1.0;
    return sign | (uint16_t)r;
  }
  const uint32_t r = a + 0xfffu + ((a >> 13) & 1);
  return sign | (uint16_t)((((r >> 23) - 112) << 10) | ((r >> 13) & 0x3ff));
}
static float round_to(int dtype, float f) {
  if (dtype == ORC_BF16) return bits_f32((uint32_t)f32_to_bf16_rne(f) << 16);
  if (dtype == ORC_F16) {
    const uint16_t h = f32_to_f16_rne(f);
    /* widen back exactly */
    const uint32_t sign = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    if (e == 0) return (sign ? -1.0f : 1.0f) * (float)m * 0x1p-24f;
    if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
    return bits_f32(sign | ((e + 112) << 23) | (m << 13));
  }
  return f;
}

static float bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* IEEE binary16 -> binary32, exact. */
static float f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1f;
  uint32_t man = h & 0x3ff;
  uint32_t u;
  if (exp == 0) {
    if (man == 0) {
      u = sign;
    } else { /* subnormal: normalise */
      int e = -1;
      do {
        man <<= 1;
        e++;
      } while ((man & 0x400) == 0);
      man &= 0x3ff;
      u = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    u = sign | 0x7f800000u | (man << 13);
  } else {
    u = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static double load_elem(const void* base, int dtype, int64_t idx) {
  if (dtype == ORC_F32) return (double)((const float*)base)[idx];
  uint16_t h = ((const uint16_t*)base)[idx];
  return dtype == ORC_BF16 ? (double)bf16_to_f32(h) : (double)f16_to_f32(h);
}

static float load_f32(const void* base, int dtype, int64_t idx) {
  if (dtype == ORC_F32) return ((const float*)base)[idx];
  uint16_t h = ((const uint16_t*)base)[idx];
  return dtype == ORC_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}

/* Element offset of (block, head, dim d, offset off) in the key cache
 * [NB, KVH, D/x, BS, x] and the value cache [NB, KVH, D, BS]. */
static int64_t key_index(int64_t blk, int head, int d, int off, int block_size, int x,
                         int64_t block_stride, int64_t head_stride) {
  return blk * block_stride + (int64_t)head * head_stride +
         ((int64_t)(d / x) * block_size + off) * x + d % x;
}
static int64_t value_index(int64_t blk, int head, int d, int off, int block_size,
                           int64_t block_stride, int64_t head_stride) {
  return blk * block_stride + (int64_t)head * head_stride + (int64_t)d * block_size + off;
}

/*
 * reshape_and_cache: for token t with s = slot_mapping[t] in
 * [0, num_blocks*block_size): blk = s / BS, off = s % BS and
 *   key_cache[blk, j, d/x, off, d%x] = key[t, j, d]
 *   value_cache[blk, j, d, off]      = value[t, j, d].
 * Bytes are copied unchanged.
 */
void oracle_reshape_and_cache(int dtype, const void* key, const void* value,
                              int64_t key_token_stride, int64_t value_token_stride,
                              void* key_cache, void* value_cache, const int64_t* slot_mapping,
                              int64_t num_tokens, int num_kv_heads, int head_dim,
                              int block_size, int64_t num_blocks, int64_t block_stride,
                              int64_t head_stride) {
  const int eb = elem_bytes(dtype);
  const int x = 16 / eb;
  for (int64_t t = 0; t < num_tokens; ++t) {
    const int64_t s = slot_mapping[t];
    if (s < 0 || s >= num_blocks * block_size) continue;
    const int64_t blk = s / block_size;
    const int off = (int)(s % block_size);
    for (int j = 0; j < num_kv_heads; ++j) {
      for (int d = 0; d < head_dim; ++d) {
        const int64_t src_k = t * key_token_stride + (int64_t)j * head_dim + d;
        const int64_t src_v = t * value_token_stride + (int64_t)j * head_dim + d;
        const int64_t dk = key_index(blk, j, d, off, block_size, x, block_stride, head_stride);
        const int64_t dv = value_index(blk, j, d, off, block_size, block_stride, head_stride);
        memcpy((char*)key_cache + dk * eb, (const char*)key + src_k * eb, eb);
        memcpy((char*)value_cache + dv * eb, (const char*)value + src_v * eb, eb);
      }
    }
  }
}

/*
 * gather_kv_cache: row cu[s] + t of out_key/out_value ([rows, KVH, D]) holds
 * token t of sequence s, read through block_tables[s, t / BS]. Blocks
 * >= num_blocks give zero rows.
 */
void oracle_gather_kv_cache(int dtype, void* out_key, void* out_value, const void* key_cache,
                            const void* value_cache, const uint32_t* block_tables,
                            int block_table_stride, const uint32_t* cu_seqlens, int num_seqs,
                            int num_kv_heads, int head_dim, int block_size, int64_t num_blocks,
                            int64_t block_stride, int64_t head_stride) {
  const int eb = elem_bytes(dtype);
  const int x = 16 / eb;
  for (int s = 0; s < num_seqs; ++s) {
    const int64_t len = (int64_t)cu_seqlens[s + 1] - cu_seqlens[s];
    for (int64_t t = 0; t < len; ++t) {
      const uint32_t blk = block_tables[(int64_t)s * block_table_stride + t / block_size];
      const int off = (int)(t % block_size);
      const int64_t row = (int64_t)cu_seqlens[s] + t;
      for (int j = 0; j < num_kv_heads; ++j) {
        for (int d = 0; d < head_dim; ++d) {
          const int64_t o = (row * num_kv_heads + j) * head_dim + d;
          if ((int64_t)blk >= num_blocks) {
            memset((char*)out_key + o * eb, 0, eb);
            memset((char*)out_value + o * eb, 0, eb);
            continue;
          }
          const int64_t sk = key_index(blk, j, d, off, block_size, x, block_stride, head_stride);
          const int64_t sv = value_index(blk, j, d, off, block_size, block_stride, head_stride);
          memcpy((char*)out_key + o * eb, (const char*)key_cache + sk * eb, eb);
          memcpy((char*)out_value + o * eb, (const char*)value_cache + sv * eb, eb);
        }
      }
    }
  }
}

/*
 * Attention of one query row against tokens [0, n_keys) of one sequence's
 * kv head, keys/values read through the paged layout, in double:
 *   s_t = scale * q . K_t   (t < n_keys and block valid)
 *   out = sum_t exp(s_t - m) V_t / (sum_t exp(s_t - m) + eps)
 * `logits` is caller scratch of n_keys doubles. Returns 0 if no token is
 * valid (out = 0).
 */
/* One cached K or V element as the attention reads it: the element itself
 * for 16/32-bit caches; for an fp8 cache (float)byte * scale rounded to the
 * query type (prefill_paged_attn.metal:764-769). */
static double load_cache(int kv_dtype, int q_dtype, const void* base, int64_t idx, float scale) {
  if (kv_dtype != ORC_FP8) return load_elem(base, kv_dtype, idx);
  return (double)round_to(q_dtype, oracle_fp8_to_f32(((const uint8_t*)base)[idx]) * scale);
}

static void attend_row_f64(int dtype, int kv_dtype, float k_scale, float v_scale, double* out,
                           const void* q, int64_t q_off, const void* key_cache,
                           const void* value_cache, const uint32_t* bt_row, int64_t n_keys,
                           int head, int head_dim, int block_size, int64_t num_blocks,
                           int64_t block_stride, int64_t head_stride, double scale, double eps,
                           double* logits) {
  const int x = 16 / elem_bytes(kv_dtype);
  double m = -INFINITY;
  for (int64_t t = 0; t < n_keys; ++t) {
    const uint32_t blk = bt_row[t / block_size];
    if ((int64_t)blk >= num_blocks) {
      logits[t] = -INFINITY;
      continue;
    }
    const int off = (int)(t % block_size);
    double acc = 0.0;
    for (int d = 0; d < head_dim; ++d)
      acc += load_elem(q, dtype, q_off + d) *
             load_cache(kv_dtype, dtype, key_cache,
                        key_index(blk, head, d, off, block_size, x, block_stride, head_stride),
                        k_scale);
    logits[t] = acc * scale;
    if (logits[t] > m) m = logits[t];
  }
  for (int d = 0; d < head_dim; ++d) out[d] = 0.0;
  if (m == -INFINITY) return;
  double sum = 0.0;
  for (int64_t t = 0; t < n_keys; ++t) {
    if (logits[t] == -INFINITY) continue;
    const double p = exp(logits[t] - m);
    sum += p;
    const uint32_t blk = bt_row[t / block_size];
    const int off = (int)(t % block_size);
    for (int d = 0; d < head_dim; ++d)
      out[d] += p * load_cache(kv_dtype, dtype, value_cache,
                               value_index(blk, head, d, off, block_size, block_stride,
                                           head_stride),
                               v_scale);
  }
  const double inv = 1.0 / (sum + eps);
  for (int d = 0; d < head_dim; ++d) out[d] *= inv;
}

/*
 * paged_attention decode, double-precision result out[num_seqs, H, D].
 * L = min(context_lens[s], max_context_len, block_table_stride * BS);
 * kv head of q head h is h / (H / KVH).
 */
void oracle_paged_attention_kv_f64(int dtype, int kv_dtype, float k_scale, float v_scale,
                                   double* out, const void* query, const void* key_cache,
                                   const void* value_cache, const uint32_t* block_tables,
                                   int block_table_stride, const uint32_t* context_lens,
                                   int max_context_len, double scale, int num_seqs,
                                   int num_heads, int num_kv_heads, int head_dim, int block_size,
                                   int64_t num_blocks, int64_t block_stride,
                                   int64_t head_stride) {
  const int group = num_heads / num_kv_heads;
#pragma omp parallel
  {
    double* logits = NULL;
    int64_t cap = 0;
#pragma omp for collapse(2) schedule(dynamic)
    for (int s = 0; s < num_seqs; ++s) {
      for (int h = 0; h < num_heads; ++h) {
        int64_t L = context_lens[s];
        if (L > max_context_len) L = max_context_len;
        if (L > (int64_t)block_table_stride * block_size)
          L = (int64_t)block_table_stride * block_size;
        if (L > cap) {
          free(logits);
          cap = L;
          logits = (double*)malloc(sizeof(double) * (size_t)cap);
        }
        attend_row_f64(dtype, kv_dtype, k_scale, v_scale,
                       out + ((int64_t)s * num_heads + h) * head_dim, query,
                       ((int64_t)s * num_heads + h) * head_dim, key_cache, value_cache,
                       block_tables + (int64_t)s * block_table_stride, L, h / group, head_dim,
                       block_size, num_blocks, block_stride, head_stride, scale, 1e-6, logits);
      }
    }
    free(logits);
  }
}

void oracle_paged_attention_f64(int dtype, double* out, const void* query,
                                const void* key_cache, const void* value_cache,
                                const uint32_t* block_tables, int block_table_stride,
                                const uint32_t* context_lens, int max_context_len, double scale,
                                int num_seqs, int num_heads, int num_kv_heads, int head_dim,
                                int block_size, int64_t num_blocks, int64_t block_stride,
                                int64_t head_stride) {
  oracle_paged_attention_kv_f64(dtype, dtype, 1.0f, 1.0f, out, query, key_cache, value_cache,
                                block_tables, block_table_stride, context_lens, max_context_len,
                                scale, num_seqs, num_heads, num_kv_heads, head_dim, block_size,
                                num_blocks, block_stride, head_stride);
}

/*
 * Chunked prefill over the paged cache, double result out[total_q, H, D].
 * Sequence s owns query rows cu_q[s] .. cu_q[s+1]-1 (n_s rows) and
 * L_s = context_lens[s] cached tokens, the last n_s of which are its own
 * rows. Query row i sits at absolute position P_s + i with P_s = L_s - n_s;
 * causal: it sees keys t <= P_s + i (attention.rs:78-149); non-causal: every
 * t < L_s (the Metal sibling kernel, prefill_paged_attn.metal:1192-1199).
 * The softmax denominator is sum + eps: 0 for the flash varlen path the CUDA
 * build takes (attention.rs:554-664), 1e-6 for the Metal kernel (:1300).
 */
void oracle_prefill_attention_kv_f64(int dtype, int kv_dtype, float k_scale, float v_scale,
                                     double* out, const void* query, const void* key_cache,
                                     const void* value_cache, const uint32_t* block_tables,
                                     int block_table_stride, const uint32_t* context_lens,
                                     const uint32_t* cu_seqlens_q, int num_seqs, int causal,
                                     double scale, int num_heads, int num_kv_heads,
                                     int head_dim, int block_size, int64_t num_blocks,
                                     int64_t block_stride, int64_t head_stride, double eps) {
  const int group = num_heads / num_kv_heads;
  for (int s = 0; s < num_seqs; ++s) {
    const int64_t n = (int64_t)cu_seqlens_q[s + 1] - cu_seqlens_q[s];
    const int64_t L = context_lens[s];
    const int64_t P = L - n;
#pragma omp parallel
    {
      double* logits = (double*)malloc(sizeof(double) * (size_t)(L > 0 ? L : 1));
#pragma omp for collapse(2) schedule(dynamic)
      for (int64_t i = 0; i < n; ++i) {
        for (int h = 0; h < num_heads; ++h) {
          const int64_t row = (int64_t)cu_seqlens_q[s] + i;
          int64_t nk = causal ? P + i + 1 : L;
          if (nk > L) nk = L;
          if (nk < 0) nk = 0;
          attend_row_f64(dtype, kv_dtype, k_scale, v_scale, out + (row * num_heads + h) * head_dim, query,
                         (row * num_heads + h) * head_dim, key_cache, value_cache,
                         block_tables + (int64_t)s * block_table_stride, nk, h / group,
                         head_dim, block_size, num_blocks, block_stride, head_stride, scale, eps,
                         logits);
        }
      }
      free(logits);
    }
  }
}

void oracle_prefill_attention_f64(int dtype, double* out, const void* query,
                                  const void* key_cache, const void* value_cache,
                                  const uint32_t* block_tables, int block_table_stride,
                                  const uint32_t* context_lens, const uint32_t* cu_seqlens_q,
                                  int num_seqs, int causal, double scale, int num_heads,
                                  int num_kv_heads, int head_dim, int block_size,
                                  int64_t num_blocks, int64_t block_stride,
                                  int64_t head_stride, double eps) {
  oracle_prefill_attention_kv_f64(dtype, dtype, 1.0f, 1.0f, out, query, key_cache, value_cache,
                                  block_tables, block_table_stride, context_lens, cu_seqlens_q,
                                  num_seqs, causal, scale, num_heads, num_kv_heads, head_dim,
                                  block_size, num_blocks, block_stride, head_stride, eps);
}

/*
 * reshape_and_cache into an fp8 cache: key/value rows of dtype `dtype`
 * ([T, KVH, D] with token strides), byte = fp8(x / scale) (see the file
 * header), layout as above with x = 16.
 */
void oracle_reshape_and_cache_fp8(int dtype, const void* key, const void* value,
                                  int64_t key_token_stride, int64_t value_token_stride,
                                  uint8_t* key_cache, uint8_t* value_cache,
                                  const int64_t* slot_mapping, int64_t num_tokens,
                                  int num_kv_heads, int head_dim, int block_size,
                                  int64_t num_blocks, int64_t block_stride, int64_t head_stride,
                                  float k_scale, float v_scale) {
  for (int64_t t = 0; t < num_tokens; ++t) {
    const int64_t s = slot_mapping[t];
    if (s < 0 || s >= num_blocks * block_size) continue;
    const int64_t blk = s / block_size;
    const int off = (int)(s % block_size);
    for (int j = 0; j < num_kv_heads; ++j) {
      for (int d = 0; d < head_dim; ++d) {
        const float k = load_f32(key, dtype, t * key_token_stride + (int64_t)j * head_dim + d);
        const float v =
            load_f32(value, dtype, t * value_token_stride + (int64_t)j * head_dim + d);
        key_cache[key_index(blk, j, d, off, block_size, 16, block_stride, head_stride)] =
            oracle_fp8_from_f32(k / k_scale);
        value_cache[value_index(blk, j, d, off, block_size, block_stride, head_stride)] =
            oracle_fp8_from_f32(v / v_scale);
      }
    }
  }
}

/*
 * gather_kv_cache from an fp8 cache: like oracle_gather_kv_cache, each value
 * dequantised to (float)byte * scale and stored as out_dtype (round to
 * nearest even); absent blocks give zero rows.
 */
void oracle_gather_kv_cache_fp8(int out_dtype, void* out_key, void* out_value,
                                const uint8_t* key_cache, const uint8_t* value_cache,
                                const uint32_t* block_tables, int block_table_stride,
                                const uint32_t* cu_seqlens, int num_seqs, int num_kv_heads,
                                int head_dim, int block_size, int64_t num_blocks,
                                int64_t block_stride, int64_t head_stride, float k_scale,
                                float v_scale) {
  const int eb = elem_bytes(out_dtype);
  for (int s = 0; s < num_seqs; ++s) {
    const int64_t len = (int64_t)cu_seqlens[s + 1] - cu_seqlens[s];
    for (int64_t t = 0; t < len; ++t) {
      const uint32_t blk = block_tables[(int64_t)s * block_table_stride + t / block_size];
      const int off = (int)(t % block_size);
      const int64_t row = (int64_t)cu_seqlens[s] + t;
      for (int j = 0; j < num_kv_heads; ++j) {
        for (int d = 0; d < head_dim; ++d) {
          const int64_t o = (row * num_kv_heads + j) * head_dim + d;
          float kf = 0.0f, vf = 0.0f;
          if ((int64_t)blk < num_blocks) {
            kf = oracle_fp8_to_f32(key_cache[key_index(blk, j, d, off, block_size, 16,
                                                       block_stride, head_stride)]) * k_scale;
            vf = oracle_fp8_to_f32(value_cache[value_index(blk, j, d, off, block_size,
                                                           block_stride, head_stride)]) * v_scale;
          }
          if (out_dtype == ORC_F32) {
            ((float*)out_key)[o] = kf;
            ((float*)out_value)[o] = vf;
          } else if (out_dtype == ORC_BF16) {
            ((uint16_t*)out_key)[o] = f32_to_bf16_rne(kf);
            ((uint16_t*)out_value)[o] = f32_to_bf16_rne(vf);
          } else {
            ((uint16_t*)out_key)[o] = f32_to_f16_rne(kf);
            ((uint16_t*)out_value)[o] = f32_to_f16_rne(vf);
          }
          (void)eb;
        }
      }
    }
  }
}

/*
 * Next-token ids of logits rows, as candle-core 0.10.2 (git rev 5404348,
 * Cargo.lock:379-381, not vendored) computes argmax over the last dim: a
 * left-to-right scan from element 0 that moves only on a strictly greater
 * value, so the first maximum wins and a NaN (never greater, never less)
 * is only kept when it is element 0. Called by the reference through
 * argmax_token_ids_from_logits (vasr-models/src/model/generation.rs:443-460).
 */
void oracle_argmax_rows(int dtype, const void* logits, int64_t row_stride, int vocab,
                        int num_rows, uint32_t* out) {
  for (int r = 0; r < num_rows; ++r) {
    const int64_t base = (int64_t)r * row_stride;
    double best = load_elem(logits, dtype, base);
    uint32_t bi = 0;
    for (int i = 1; i < vocab; ++i) {
      const double v = load_elem(logits, dtype, base + i);
      if (v > best) {
        best = v;
        bi = (uint32_t)i;
      }
    }
    out[r] = bi;
  }
}

/*
 * Step-start bookkeeping of paged_batch_decode_step
 * (vasr-models/src/model/paged_batch_engine.rs:640-667) over per-row state:
 * a row that is not finished takes its pending id; an EOS id finishes it,
 * any other id is appended to its generated list (up to gen_capacity) and
 * becomes its input id. Finished rows get eos_fill_id as input (the
 * reference's pad id, eos_token_ids[0], paged_batch_engine.rs:193-195).
 * *active_count = rows that fed a real token. With prev_slots (the
 * previous step's slot_mapping), an unfinished row whose previous slot is
 * negative did not run: it feeds input_ids[r] again and consumes nothing
 * (the reference keeps a slot that could not allocate out of the forward
 * with its pending id, paged_batch_engine.rs:209-227).
 */
void oracle_decode_consume_tokens(const uint32_t* next_ids, uint8_t* finished,
                                  const int64_t* prev_slots, uint32_t* generated,
                                  uint32_t* gen_len, int gen_capacity,
                                  const uint32_t* eos_ids, int num_eos, uint32_t eos_fill_id,
                                  uint32_t* input_ids, uint32_t* active_count, int num_rows) {
  uint32_t active = 0;
  for (int r = 0; r < num_rows; ++r) {
    uint32_t feed = eos_fill_id;
    if (!finished[r] && prev_slots != NULL && prev_slots[r] < 0) {
      feed = input_ids[r];
      ++active;
    } else if (!finished[r]) {
      const uint32_t tok = next_ids[r];
      int eos = 0;
      for (int e = 0; e < num_eos; ++e) eos |= tok == eos_ids[e];
      if (eos) {
        finished[r] = 1;
      } else {
        if ((int64_t)gen_len[r] < gen_capacity) {
          generated[(int64_t)r * gen_capacity + gen_len[r]] = tok;
          gen_len[r] += 1;
        }
        feed = tok;
        ++active;
      }
    }
    input_ids[r] = feed;
  }
  *active_count = active;
}

/* ---------------------------------------------------------------------- */
/* CPU baseline: the reference's CPU decode path restated in f32.           */
/* ---------------------------------------------------------------------- */

/*
 * One decode step for `num_seqs` sequences of one layer, as the reference's
 * CPU path would run it over the paged data:
 *   1. append the new token's K/V at slot_mapping[s] (reshape_and_cache
 *      semantics; the CPU path's contiguous append is kv_cache.rs:54-111);
 *   2. per (sequence, kv head): gather the L_s cached rows into a contiguous
 *      buffer (the contiguous (kvh, L, D) cache of the CPU path), then for
 *      each query head of the group QK^T * scale -> softmax -> .V
 *      (repeat_kv + attention.rs:243-286).
 * out is [num_seqs, H, D] f32. Returns the number of OpenMP threads used.
 */
int cpu_baseline_decode_step(int dtype, float* out, const void* query, const void* new_key,
                             const void* new_value, const int64_t* slot_mapping, void* key_cache,
                             void* value_cache, const uint32_t* block_tables,
                             int block_table_stride, const uint32_t* context_lens,
                             float scale, int num_seqs, int num_heads, int num_kv_heads,
                             int head_dim, int block_size, int64_t num_blocks,
                             int64_t block_stride, int64_t head_stride) {
  const int x = 16 / elem_bytes(dtype);
  const int group = num_heads / num_kv_heads;
  const int64_t row = (int64_t)num_kv_heads * head_dim;
  oracle_reshape_and_cache(dtype, new_key, new_value, row, row, key_cache, value_cache,
                           slot_mapping, num_seqs, num_kv_heads, head_dim, block_size,
                           num_blocks, block_stride, head_stride);
  int threads = 1;
#pragma omp parallel
  {
#ifdef _OPENMP
#pragma omp single
    threads = omp_get_num_threads();
#endif
    float* kbuf = NULL;
    float* vbuf = NULL;
    float* logits = NULL;
    int64_t cap = 0;
#pragma omp for collapse(2) schedule(dynamic)
    for (int s = 0; s < num_seqs; ++s) {
      for (int j = 0; j < num_kv_heads; ++j) {
        const int64_t L = context_lens[s];
        if (L > cap) {
          free(kbuf);
          free(vbuf);
          free(logits);
          cap = L;
          kbuf = (float*)malloc(sizeof(float) * (size_t)(cap * head_dim));
          vbuf = (float*)malloc(sizeof(float) * (size_t)(cap * head_dim));
          logits = (float*)malloc(sizeof(float) * (size_t)cap);
        }
        const uint32_t* bt = block_tables + (int64_t)s * block_table_stride;
        for (int64_t t = 0; t < L; ++t) {
          const int64_t blk = bt[t / block_size];
          const int off = (int)(t % block_size);
          for (int d = 0; d < head_dim; ++d) {
            kbuf[t * head_dim + d] = load_f32(
                key_cache, dtype, key_index(blk, j, d, off, block_size, x, block_stride, head_stride));
            vbuf[t * head_dim + d] = load_f32(
                value_cache, dtype, value_index(blk, j, d, off, block_size, block_stride, head_stride));
          }
        }
        for (int g = 0; g < group; ++g) {
          const int h = j * group + g;
          const int64_t qo = ((int64_t)s * num_heads + h) * head_dim;
          float m = -INFINITY;
          for (int64_t t = 0; t < L; ++t) {
            float acc = 0.f;
            for (int d = 0; d < head_dim; ++d)
              acc += load_f32(query, dtype, qo + d) * kbuf[t * head_dim + d];
            logits[t] = acc * scale;
            if (logits[t] > m) m = logits[t];
          }
          float sum = 0.f;
          for (int64_t t = 0; t < L; ++t) {
            logits[t] = expf(logits[t] - m);
            sum += logits[t];
          }
          float* o = out + qo;
          for (int d = 0; d < head_dim; ++d) o[d] = 0.f;
          for (int64_t t = 0; t < L; ++t) {
            const float p = logits[t] / sum;
            for (int d = 0; d < head_dim; ++d) o[d] += p * vbuf[t * head_dim + d];
          }
        }
      }
    }
    free(kbuf);
    free(vbuf);
    free(logits);
  }
  return threads;
}
