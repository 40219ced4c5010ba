// Next-token selection and EOS state of the decode loop, kept on the GPU
// (gfx950).
//
// The reference picks next tokens on the host: argmax over each row of the
// step's logits (vasr-models/src/model/generation.rs:443-460, candle's
// argmax), a read-back of every id, then the step-start bookkeeping of
// paged_batch_decode_step (vasr-models/src/model/paged_batch_engine.rs:
// 640-667): a row whose pending token is an EOS id becomes finished and is
// dropped; every other row appends its pending token to its generated list
// and feeds it as the next input id. Its own notes measure that per-step
// read-back as the largest decode cost (docs/performance/qwen3-asr-cuda-graph-
// raw-audios-bottleneck-notes.md:373-401, 700-730) and propose the device
// version built here: ids and finished flags stay in device buffers,
// finished rows feed the EOS fill id (eos_token_ids[0], as the slot decode
// path pads, paged_batch_engine.rs:193-195) instead of being compacted out,
// and the host reads one 4-byte active count only when it wants to stop.
//
// argmax_rows_kernel: one 1024-thread workgroup per row; 16-byte loads of the
// row (four in flight per thread), a per-thread best (value, index), then
// wave and workgroup reductions.
// Candle's argmax scans left to right and moves only on a strictly greater
// value: the first maximum wins, a NaN is never taken after element 0, and
// a NaN at element 0 is never left. The reduction keeps exactly that order:
// ties go to the lower index, NaNs are skipped, and element 0 being NaN
// gives 0.
//
// consume_tokens_kernel: one workgroup walks the rows (the state is small)
// and counts the rows that fed a real token.

#include <math.h>

#include "vpa_device.h"
#include "vpa_internal.h"

namespace vpa {
namespace {

constexpr int kArgmaxThreads = 1024;

// (value, index) a is better than b: greater, or equal with a lower index.
__device__ __forceinline__ bool better(float av, uint32_t ai, float bv, uint32_t bi) {
  return av > bv || (av == bv && ai < bi);
}

template <typename T>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_rows_kernel(
    const T* __restrict__ logits, int64_t row_stride, int32_t vocab, uint32_t* __restrict__ out,
    int32_t vec_ok) {
  constexpr int X = pack_x<T>();
  __shared__ float s_v[kArgmaxThreads / 64];
  __shared__ uint32_t s_i[kArgmaxThreads / 64];
  const int tid = threadIdx.x;
  const T* row = logits + (int64_t)blockIdx.x * row_stride;
  float bv = -INFINITY;
  uint32_t bi = 0xffffffffu;
  auto take = [&](float v, uint32_t i) {
    if (!isnan(v) && better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  };
  int v0 = 0;
  if (vec_ok) {
    // four non-temporal 16-byte loads in flight per thread (the logits are
    // read once); the result does not depend on the order of the takes
    const int nvec = vocab / X;
    const uint4* rv = reinterpret_cast<const uint4*>(row);
    auto take_vec = [&](const uint4& u, int q) {
      const T* e = reinterpret_cast<const T*>(&u);
#pragma unroll
      for (int k = 0; k < X; ++k) take(load_as_f32(e + k), (uint32_t)(q * X + k));
    };
    int q = tid;
    for (; q + 3 * kArgmaxThreads < nvec; q += 4 * kArgmaxThreads) {
      uint4 u[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) u[j] = load_stream(rv + q + j * kArgmaxThreads);
#pragma unroll
      for (int j = 0; j < 4; ++j) take_vec(u[j], q + j * kArgmaxThreads);
    }
    for (; q < nvec; q += kArgmaxThreads) take_vec(load_stream(rv + q), q);
    v0 = nvec * X;
  }
  for (int i = v0 + tid; i < vocab; i += kArgmaxThreads) take(load_as_f32(row + i), (uint32_t)i);
  // wave, then workgroup
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const uint32_t oi = __shfl_xor(bi, off, 64);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if ((tid & 63) == 0) {
    s_v[tid >> 6] = bv;
    s_i[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kArgmaxThreads / 64; ++w)
      if (better(s_v[w], s_i[w], bv, bi)) {
        bv = s_v[w];
        bi = s_i[w];
      }
    // element 0 NaN: a left-to-right strict-greater scan never leaves it;
    // an all-NaN row likewise ends at 0
    if (isnan(load_as_f32(row)) || bi == 0xffffffffu) bi = 0;
    out[blockIdx.x] = bi;
  }
}

constexpr int kConsumeThreads = 1024;

__global__ __launch_bounds__(kConsumeThreads) void consume_tokens_kernel(
    const uint32_t* __restrict__ next_ids, uint8_t* __restrict__ finished,
    const int64_t* __restrict__ prev_slots, uint32_t* __restrict__ generated, uint32_t* __restrict__ gen_len, int32_t gen_capacity,
    const uint32_t* __restrict__ eos_ids, int32_t num_eos, uint32_t eos_fill_id,
    uint32_t* __restrict__ input_ids, uint32_t* __restrict__ active_count, int32_t num_rows) {
  __shared__ uint32_t s_cnt[kConsumeThreads / 64];
  const int tid = threadIdx.x;
  uint32_t active = 0;
  for (int r = tid; r < num_rows; r += kConsumeThreads) {
    uint32_t feed = eos_fill_id;
    if (!finished[r] && prev_slots != nullptr && prev_slots[r] < 0) {
      // the previous step did not run this row (no block for its token): it
      // feeds the same input again and its pending id is stale
      feed = input_ids[r];
      ++active;
    } else if (!finished[r]) {
      const uint32_t tok = next_ids[r];
      bool eos = false;
      for (int e = 0; e < num_eos; ++e) eos = eos || tok == eos_ids[e];
      if (eos) {
        finished[r] = 1;
      } else {
        const uint32_t n = gen_len[r];
        if ((int64_t)n < gen_capacity) {
          generated[(int64_t)r * gen_capacity + n] = tok;
          gen_len[r] = n + 1;
        }
        feed = tok;
        ++active;
      }
    }
    input_ids[r] = feed;
  }
  // workgroup sum of the active rows
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) active += __shfl_xor(active, off, 64);
  if ((tid & 63) == 0) s_cnt[tid >> 6] = active;
  __syncthreads();
  if (tid == 0) {
    uint32_t t = 0;
    for (int w = 0; w < kConsumeThreads / 64; ++w) t += s_cnt[w];
    *active_count = t;
  }
}

}  // namespace

hipError_t launch_argmax_rows(int dtype, const void* logits, int64_t row_stride, int32_t vocab,
                              int32_t num_rows, uint32_t* out, hipStream_t stream) {
  const int eb = dtype == VPA_DTYPE_F32 ? 4 : 2;
  const bool vec_ok = (reinterpret_cast<uintptr_t>(logits) & 15u) == 0 && (row_stride * eb) % 16 == 0;
  if (dtype == VPA_DTYPE_F32)
    hipLaunchKernelGGL(argmax_rows_kernel<float>, dim3(num_rows), dim3(kArgmaxThreads), 0,
                       stream, static_cast<const float*>(logits), row_stride, vocab, out,
                       (int32_t)vec_ok);
  else if (dtype == VPA_DTYPE_BF16)
    hipLaunchKernelGGL(argmax_rows_kernel<bf16_t>, dim3(num_rows), dim3(kArgmaxThreads), 0,
                       stream, static_cast<const bf16_t*>(logits), row_stride, vocab, out,
                       (int32_t)vec_ok);
  else if (dtype == VPA_DTYPE_F16)
    hipLaunchKernelGGL(argmax_rows_kernel<f16_t>, dim3(num_rows), dim3(kArgmaxThreads), 0,
                       stream, static_cast<const f16_t*>(logits), row_stride, vocab, out,
                       (int32_t)vec_ok);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_consume_tokens(const uint32_t* next_ids, uint8_t* finished,
                                 const int64_t* prev_slot_mapping, uint32_t* generated, uint32_t* gen_len, int32_t gen_capacity,
                                 const uint32_t* eos_ids, int32_t num_eos, uint32_t eos_fill_id,
                                 uint32_t* input_ids, uint32_t* active_count, int32_t num_rows,
                                 hipStream_t stream) {
  hipLaunchKernelGGL(consume_tokens_kernel, dim3(1), dim3(kConsumeThreads), 0, stream, next_ids,
                     finished, prev_slot_mapping, generated, gen_len, gen_capacity, eos_ids, num_eos, eos_fill_id,
                     input_ids, active_count, num_rows);
  return hipGetLastError();
}

}  // namespace vpa
