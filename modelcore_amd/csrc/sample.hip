// Next-token sampling on the device with a counter-based RNG per row.
//
// Row b draws token argmax_i (logits[b, i] / T + g_i), where g_i = -log(-log(u_i)) is standard
// Gumbel noise and u_i is uniform in (0, 1): the Gumbel-max form of sampling from
// softmax(logits[b] / T), the distribution modelcore/generate.py:18-34 draws from with
// torch.multinomial. T == 0 takes the plain argmax (greedy), as the reference does. Ties go to
// the lowest index, as torch.argmax does.
//
// The uniforms come from Philox4x32-10 (Salmon, Moraes, Dror and Shaw, "Parallel random numbers:
// as easy as 1, 2, 3", SC 2011): key = the row's 64-bit seed, counter = (i / 4, row offset,
// 0, 0), word i % 4; u = ((x >> 9) + 1/2) / 2^23, an exact float32 in (0, 1). Each call
// consumes one offset per row and advances offsets[b] by one on the device, so a row's draws
// depend only on its seed and on how many tokens it has drawn -- never on the batch it sits in
// -- and no host sync is needed.
//
// One workgroup per row; each lane scans a strided part of the vocabulary, then a wave64
// reduction and an LDS reduction over the waves pick the (score, index) maximum.
#include "kernels.h"

#include <cmath>

namespace mcamd {
namespace {

constexpr int kThreads = 256;

struct Philox {
  uint32_t c0, c1, c2, c3;
};

// Philox4x32 with 10 rounds on counter (c0..c3) and key (k0, k1).
__device__ __forceinline__ Philox philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                                uint32_t k0, uint32_t k1) {
  constexpr uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u;  // round multipliers
  constexpr uint32_t W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;  // key schedule increments
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint32_t hi0 = __umulhi(M0, c0), lo0 = M0 * c0;
    const uint32_t hi1 = __umulhi(M1, c2), lo1 = M1 * c2;
    const uint32_t n0 = hi1 ^ c1 ^ k0, n1 = lo1, n2 = hi0 ^ c3 ^ k1, n3 = lo0;
    c0 = n0;
    c1 = n1;
    c2 = n2;
    c3 = n3;
    k0 += W0;
    k1 += W1;
  }
  return {c0, c1, c2, c3};
}

// (k + 1/2) / 2^23 for the top 23 bits k of x: exactly representable, strictly inside (0, 1).
__device__ __forceinline__ float uniform23(uint32_t x) {
  return (float(x >> 9) + 0.5f) * (1.0f / 8388608.0f);
}

__device__ __forceinline__ bool better(float s, int i, float bs, int bi) {
  return s > bs || (s == bs && i < bi);
}

__global__ __launch_bounds__(kThreads) void sample_kernel(const float *__restrict__ logits,
                                                          int64_t row_stride, int vocab,
                                                          float inv_temp, int greedy,
                                                          const uint64_t *__restrict__ seeds,
                                                          int64_t *__restrict__ offsets,
                                                          int64_t *__restrict__ out) {
  __shared__ float s_score[kThreads / 64];
  __shared__ int s_index[kThreads / 64];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const float *row = logits + int64_t(b) * row_stride;
  const uint64_t seed = seeds[b];
  const uint64_t off = uint64_t(offsets[b]);
  const uint32_t k0 = uint32_t(seed), k1 = uint32_t(seed >> 32);
  float best = -INFINITY;
  int best_i = 0x7fffffff;
  // Lane tid handles groups of four consecutive tokens 4 g .. 4 g + 3, g = tid, tid + 256, ...
  for (int g = tid; 4 * g < vocab; g += kThreads) {
    Philox r{0, 0, 0, 0};
    if (!greedy) r = philox4x32_10(uint32_t(g), uint32_t(off), uint32_t(off >> 32), 0u, k0, k1);
    const uint32_t w[4] = {r.c0, r.c1, r.c2, r.c3};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = 4 * g + j;
      if (i >= vocab) break;
      float s = row[i];
      if (!greedy) s = s * inv_temp - logf(-logf(uniform23(w[j])));
      if (s != s) s = -INFINITY;  // a NaN logit never wins
      if (better(s, i, best, best_i)) {
        best = s;
        best_i = i;
      }
    }
  }
  // (score, index) maximum over the wave, then over the workgroup.
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float os = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(best_i, o, 64);
    if (better(os, oi, best, best_i)) {
      best = os;
      best_i = oi;
    }
  }
  if ((tid & 63) == 0) {
    s_score[tid >> 6] = best;
    s_index[tid >> 6] = best_i;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kThreads / 64; ++w)
      if (better(s_score[w], s_index[w], best, best_i)) {
        best = s_score[w];
        best_i = s_index[w];
      }
    out[b] = best_i == 0x7fffffff ? 0 : best_i;
    offsets[b] = int64_t(off + 1);
  }
}

}  // namespace
}  // namespace mcamd

using namespace mcamd;

extern "C" int mcamd_sample_tokens(const float *logits, int64_t batch, int64_t vocab,
                                   int64_t row_stride, float temperature, const uint64_t *seeds,
                                   int64_t *offsets, int64_t *out, void *stream) {
  if (batch < 0 || vocab <= 0 || vocab > (int64_t(1) << 30) || (row_stride != 0 && row_stride < vocab))
    return fail(MCAMD_EINVAL,
                "sample_tokens: need batch >= 0, 0 < vocab <= 2^30, row_stride 0 or >= vocab");
  if (!(temperature >= 0.f) || std::isinf(temperature))
    return fail(MCAMD_EINVAL, "sample_tokens: temperature must be finite and non-negative");
  if (batch > 0 && (!logits || !seeds || !offsets || !out))
    return fail(MCAMD_EINVAL, "sample_tokens: null pointer");
  if (batch > 0x7fffffff) return fail(MCAMD_EUNSUPPORTED, "sample_tokens: batch too large");
  if (batch == 0) {
    clear_error();
    return MCAMD_OK;
  }
  const int greedy = temperature == 0.f ? 1 : 0;
  const float inv_temp = greedy ? 1.f : 1.f / temperature;
  hipLaunchKernelGGL(sample_kernel, dim3(unsigned(batch)), dim3(kThreads), 0, as_stream(stream),
                     logits, row_stride, int(vocab), inv_temp, greedy, seeds, offsets, out);
  return launch_status("sample_tokens");
}
