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
// reduction and an LDS reduction over the waves pick the (score, index) maximum. The result does
// not depend on the workgroup size: a token's noise is keyed by its own index.
//
// top_k (0 < k < vocab) restricts the draw to the k largest logits, ties at the k-th value going
// to the lowest indices -- the set torch.topk returns for distinct values -- and the Gumbel-max
// over that set is a draw from softmax(top-k logits / T), the distribution of the reference's
// top_k branch. The k-th largest value is found without sorting: logits map to 32-bit keys in
// the same order (NaN lowest), and a binary search over the key bits counts, for each candidate,
// the row's keys at or above it (one block-wide count per bit, the row held in registers when it
// fits, else re-read from the cache hierarchy).
#include "kernels.h"

#include <cmath>

namespace mcamd {
namespace {

constexpr int kThreads = 256;
// The plain draw: sixteen waves per row, so that the Philox rounds and logarithms of a row (its
// cost; one row per CU) run on every SIMD with four waves each to interleave (measured on the
// 64-row, 32768-token sampling step: 31.5 -> 18.1 us per draw against four waves).
constexpr int kDrawThreads = 1024;

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

// A 32-bit key in the order of the float (NaN below everything, -inf next; -0 equal to +0).
__device__ __forceinline__ uint32_t order_key(float f) {
  if (f != f) return 0u;
  uint32_t u = __float_as_uint(f);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Sum of one int per thread over the workgroup; `slot` alternates between calls so that one
// barrier per call suffices.
__device__ __forceinline__ int block_sum(int v, int (*s_cnt)[kThreads / 64], int &slot) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  if ((threadIdx.x & 63) == 0) s_cnt[slot][threadIdx.x >> 6] = v;
  __syncthreads();
  int t = 0;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) t += s_cnt[slot][w];
  slot ^= 1;
  return t;
}

constexpr int kRegGroups = 32;  // groups of four logits a thread holds in registers (vocab <= 32768)

__global__ __launch_bounds__(kDrawThreads) void sample_kernel(const float *__restrict__ logits,
                                                          int64_t row_stride, int vocab,
                                                          float inv_temp, int greedy,
                                                          const uint64_t *__restrict__ seeds,
                                                          int64_t *__restrict__ offsets,
                                                          int64_t *__restrict__ out) {
  __shared__ float s_score[kDrawThreads / 64];
  __shared__ int s_index[kDrawThreads / 64];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const float *row = logits + int64_t(b) * row_stride;
  const uint64_t seed = seeds[b];
  const uint64_t off = uint64_t(offsets[b]);
  const uint32_t k0 = uint32_t(seed), k1 = uint32_t(seed >> 32);
  float best = -INFINITY;
  int best_i = 0x7fffffff;
  // Lane tid handles groups of four consecutive tokens 4 g .. 4 g + 3, g = tid, tid + 256, ...
  for (int g = tid; 4 * g < vocab; g += kDrawThreads) {
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
    for (int w = 1; w < kDrawThreads / 64; ++w)
      if (better(s_score[w], s_index[w], best, best_i)) {
        best = s_score[w];
        best_i = s_index[w];
      }
    out[b] = best_i == 0x7fffffff ? 0 : best_i;
    offsets[b] = int64_t(off + 1);
  }
}

// The draw restricted to the top_k largest logits of the row (see the top of the file). REG: the
// row is held in registers (vocab <= 4 * kThreads * kRegGroups), else read again for every count.
template <bool REG>
__global__ __launch_bounds__(kThreads) void sample_topk_kernel(const float *__restrict__ logits,
                                                               int64_t row_stride, int vocab,
                                                               int top_k, float inv_temp,
                                                               const uint64_t *__restrict__ seeds,
                                                               int64_t *__restrict__ offsets,
                                                               int64_t *__restrict__ out) {
  __shared__ int s_cnt[2][kThreads / 64];
  __shared__ float s_score[kThreads / 64];
  __shared__ int s_index[kThreads / 64];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  const float *row = logits + int64_t(b) * row_stride;
  const int n_groups = (vocab + 3) / 4;
  // The row's keys: in registers (thread tid holds groups tid + m * kThreads; past the vocabulary
  // the key is 0, which no candidate below reaches), or read from memory for each count.
  constexpr int NK = REG ? 4 * kRegGroups : 1;
  uint32_t key[NK];
  if constexpr (REG) {
#pragma unroll
    for (int m = 0; m < kRegGroups; ++m)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = 4 * (tid + m * kThreads) + j;
        key[4 * m + j] = i < vocab ? order_key(row[i]) : 0u;
      }
  }
  int slot = 0;
  // Block-wide counts of keys >= c, > c, == c, and == c at an index below `below`.
  auto count_ge = [&](uint32_t c) {
    int n = 0;
    if constexpr (REG) {
#pragma unroll
      for (int e = 0; e < NK; ++e) n += key[e] >= c ? 1 : 0;
    } else {
      for (int i = tid; i < vocab; i += kThreads) n += order_key(row[i]) >= c ? 1 : 0;
    }
    return block_sum(n, s_cnt, slot);
  };
  auto count_eq_below = [&](uint32_t c, int below) {
    int n = 0;
    if constexpr (REG) {
#pragma unroll
      for (int m = 0; m < kRegGroups; ++m)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          n += (key[4 * m + j] == c && 4 * (tid + m * kThreads) + j < below) ? 1 : 0;
    } else {
      for (int i = tid; i < vocab && i < below; i += kThreads) n += order_key(row[i]) == c ? 1 : 0;
    }
    return block_sum(n, s_cnt, slot);
  };
  // K = the k-th largest key: the largest K with at least k keys >= K (every candidate is >= 1).
  uint32_t K = 0;
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t cand = K | (1u << bit);
    if (count_ge(cand) >= top_k) K = cand;
  }
  // Keys equal to K past the k-th position are left out: the lowest-index ones are kept.
  const int above = K == 0xffffffffu ? 0 : count_ge(K + 1);
  const int ties = count_eq_below(K, 0x7fffffff);
  const int need = top_k - above;  // 1 <= need <= ties
  int last_tie = 0x7fffffff;       // highest index among the kept ties
  if (need < ties) {
    int lo = 0;  // the largest index with fewer than `need` ties below it is the last kept tie
    for (int bit = 30; bit >= 0; --bit) {
      const int cand = lo | (1 << bit);
      if (count_eq_below(K, cand) < need) lo = cand;
    }
    last_tie = lo;
  }

  const uint64_t seed = seeds[b];
  const uint64_t off = uint64_t(offsets[b]);
  const uint32_t k0 = uint32_t(seed), k1 = uint32_t(seed >> 32);
  float best = -INFINITY;
  int best_i = 0x7fffffff;
  // Gumbel-max over the kept logits of group g (four consecutive tokens, one Philox counter).
  auto group = [&](int g, const float (&v)[4]) {
    const Philox r = philox4x32_10(uint32_t(g), uint32_t(off), uint32_t(off >> 32), 0u, k0, k1);
    const uint32_t w[4] = {r.c0, r.c1, r.c2, r.c3};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = 4 * g + j;
      const uint32_t key = order_key(v[j]);
      if (i >= vocab || !(key > K || (key == K && i <= last_tie))) continue;
      float sc = v[j] * inv_temp - logf(-logf(uniform23(w[j])));
      if (sc != sc) sc = -INFINITY;
      if (better(sc, i, best, best_i)) {
        best = sc;
        best_i = i;
      }
    }
  };
  for (int g = tid; g < n_groups; g += kThreads) {
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = 4 * g + j < vocab ? row[4 * g + j] : 0.f;
    group(g, v);
  }
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
                                   int64_t row_stride, float temperature, int64_t top_k,
                                   const uint64_t *seeds, int64_t *offsets, int64_t *out,
                                   void *stream) {
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
  if (!greedy && top_k > 0 && top_k < vocab) {
    if (vocab <= int64_t(4) * kThreads * kRegGroups)
      hipLaunchKernelGGL(sample_topk_kernel<true>, dim3(unsigned(batch)), dim3(kThreads), 0,
                         as_stream(stream), logits, row_stride, int(vocab), int(top_k), inv_temp,
                         seeds, offsets, out);
    else
      hipLaunchKernelGGL(sample_topk_kernel<false>, dim3(unsigned(batch)), dim3(kThreads), 0,
                         as_stream(stream), logits, row_stride, int(vocab), int(top_k), inv_temp,
                         seeds, offsets, out);
    return launch_status("sample_tokens (top_k)");
  }
  hipLaunchKernelGGL(sample_kernel, dim3(unsigned(batch)), dim3(kDrawThreads), 0, as_stream(stream),
                     logits, row_stride, int(vocab), inv_temp, greedy, seeds, offsets, out);
  return launch_status("sample_tokens");
}
