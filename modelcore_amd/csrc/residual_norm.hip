// The residual update and the RMS-norm after a projection, fused, for decode-sized batches:
//   y      = bf16(sum over s of part[s][m][:])        (the K-split partials of the projection, in
//                                                     order; or y given in bf16)
//   x_out  = bf16(x + y)                               (the residual stream, `x = x + f(norm(x))`)
//   h_out  = bf16(x_out * rsqrt(mean(x_out^2) + eps))  (the next norm, fp32 arithmetic)
// Replaces, per block of the reference (modelcore/components/block.py:54-60), the split-K reduce
// of the projection, the residual add and the following RMSNorm (modelcore/components/norm.py:
// 43-44, F.rms_norm): three launches become one, and h_out feeds the next projection (or the
// next block's mixer, or the lm_head) directly.
//
// One workgroup of 256 threads per row m; each thread owns chunks of 8 elements (16 bytes of
// bf16, 32 of fp32 partials), so every load and store is a full 16-byte vector, and keeps them in
// registers between the sum and the norm (rows up to 8192 elements). The mean square is a wave
// sum (shuffles) then a sum over the four waves through LDS.
#include "kernels.h"

namespace mcamd {
namespace {

constexpr int kThreads = 256;
// Partial counts whose loads are issued together: up to this many for any row that fits the
// registers, up to twice as many for rows of at most 2 * kThreads chunks (4096 elements).
constexpr int kMaxBatchedSplits = 4;

struct ResParams {
  const uint16_t *x, *y;
  const float *part;
  uint16_t *x_out, *h_out;
  int M, N, S;
  float eps;
};

__device__ __forceinline__ uint16_t to_bf16(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}
__device__ __forceinline__ float bf16_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }
__device__ __forceinline__ void unpack8(const uint4 &u, float (&v)[8]) {
  v[0] = bf16_lo(u.x), v[1] = bf16_hi(u.x), v[2] = bf16_lo(u.y), v[3] = bf16_hi(u.y);
  v[4] = bf16_lo(u.z), v[5] = bf16_hi(u.z), v[6] = bf16_lo(u.w), v[7] = bf16_hi(u.w);
}
__device__ __forceinline__ uint4 pack8(const float (&v)[8]) {
  return uint4{uint32_t(to_bf16(v[0])) | (uint32_t(to_bf16(v[1])) << 16),
               uint32_t(to_bf16(v[2])) | (uint32_t(to_bf16(v[3])) << 16),
               uint32_t(to_bf16(v[4])) | (uint32_t(to_bf16(v[5])) << 16),
               uint32_t(to_bf16(v[6])) | (uint32_t(to_bf16(v[7])) << 16)};
}

// CPT > 0: each thread keeps its (at most CPT) chunks of x_out in registers for the norm;
// CPT = 0: any row length, the norm pass re-reads the thread's own chunks of x_out.
// MAXS > 0 (at most MAXS partials): the partial loads of all the thread's chunks are issued
// before the first is summed, so they cost one memory latency, not one per partial and chunk;
// MAXS = 0: any number of partials, loaded one after the other.
// The fields of ResParams come as separate scalar arguments: the library is built with kernarg
// preloading (leading scalar arguments, as many as fit the 14 free user SGPRs), and these
// fourteen dwords all arrive in SGPRs at dispatch.
template <int CPT, int MAXS>
__global__ __launch_bounds__(kThreads) void residual_rmsnorm_kernel(
    const uint16_t *a_x, const uint16_t *a_y, const float *a_part, uint16_t *a_x_out,
    uint16_t *a_h_out, int a_M, int a_N, int a_S, float a_eps) {
  ResParams P;
  P.x = a_x;
  P.y = a_y;
  P.part = a_part;
  P.x_out = a_x_out;
  P.h_out = a_h_out;
  P.M = a_M;
  P.N = a_N;
  P.S = a_S;
  P.eps = a_eps;
  __shared__ float wsum[kThreads / 64];
  const int m = blockIdx.x;
  const int chunks = P.N / 8;
  const int64_t row = int64_t(m) * P.N;
  constexpr int kHeld = CPT > 0 ? CPT : 1;
  float held[kHeld][8];
  float ss = 0.f;
  // A chunk's inputs: x, and y or (with MAXS > 0) the partials. All of a thread's chunks are
  // loaded before the first is summed and stored (x_out may be x itself, so the compiler would
  // not move a later chunk's loads above an earlier chunk's store on its own).
  constexpr int kS = MAXS > 0 ? MAXS : 1;
  uint4 xin[kHeld], yin[kHeld];
  float4 pa[kHeld][kS], pb[kHeld][kS];
  auto slice = [&](int s, int c) {
    return reinterpret_cast<const float4 *>(P.part + int64_t(s) * P.M * P.N + row + 8 * c);
  };
  // The loads of chunk c into slot u. With MAXS > 0 the last partial stands in for absent ones
  // (the sum skips them), so every load issues here.
  auto load_x = [&](int c, int u) { xin[u] = *reinterpret_cast<const uint4 *>(P.x + row + 8 * c); };
  auto load_y = [&](int c, int u) { yin[u] = *reinterpret_cast<const uint4 *>(P.y + row + 8 * c); };
  auto load_parts = [&](int c, int u) {
    if constexpr (MAXS > 0) {
#pragma unroll
      for (int s = 0; s < MAXS; ++s) {
        const float4 *q = slice(min(s, P.S - 1), c);
        pa[u][s] = q[0], pb[u][s] = q[1];
      }
    }
  };
  // All slots' loads, unconditional (a slot past the row re-reads its last chunk) and in one
  // block per input kind, so that no arithmetic is scheduled between them.
  auto load_all = [&]() {
#pragma unroll
    for (int u = 0; u < CPT; ++u) load_x(min(int(threadIdx.x) + u * kThreads, chunks - 1), u);
    if (P.part) {
#pragma unroll
      for (int u = 0; u < CPT; ++u) load_parts(min(int(threadIdx.x) + u * kThreads, chunks - 1), u);
    } else {
#pragma unroll
      for (int u = 0; u < CPT; ++u) load_y(min(int(threadIdx.x) + u * kThreads, chunks - 1), u);
    }
  };
  auto residual_chunk = [&](int c, int u, float (&sv)[8]) {
    float xv[8], yv[8];
    unpack8(xin[u], xv);
    if (P.part) {
      // The in-order fp32 sum of the partials, as the GEMM's own reduce pass makes it.
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if constexpr (MAXS > 0) {
#pragma unroll
        for (int s = 0; s < MAXS; ++s) {
          if (s < P.S) {
            acc[0] += pa[u][s].x, acc[1] += pa[u][s].y, acc[2] += pa[u][s].z, acc[3] += pa[u][s].w;
            acc[4] += pb[u][s].x, acc[5] += pb[u][s].y, acc[6] += pb[u][s].z, acc[7] += pb[u][s].w;
          }
        }
      } else {
        for (int s = 0; s < P.S; ++s) {
          const float4 a = slice(s, c)[0], b = slice(s, c)[1];
          acc[0] += a.x, acc[1] += a.y, acc[2] += a.z, acc[3] += a.w;
          acc[4] += b.x, acc[5] += b.y, acc[6] += b.z, acc[7] += b.w;
        }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) yv[i] = __uint_as_float(uint32_t(to_bf16(acc[i])) << 16);
    } else {
      unpack8(yin[u], yv);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      sv[i] = __uint_as_float(uint32_t(to_bf16(xv[i] + yv[i])) << 16);
      ss = fmaf(sv[i], sv[i], ss);
    }
    *reinterpret_cast<uint4 *>(P.x_out + row + 8 * c) = pack8(sv);
  };
  if constexpr (CPT > 0) {
    load_all();
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int c = threadIdx.x + u * kThreads;
      if (c < chunks) residual_chunk(c, u, held[u]);
    }
  } else {
    for (int c = threadIdx.x; c < chunks; c += kThreads) {
      load_x(c, 0);
      if (P.part)
        load_parts(c, 0);
      else
        load_y(c, 0);
      residual_chunk(c, 0, held[0]);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
  if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = ss;
  lds_barrier();  // the x_out stores above need not land before the norm's sum is shared
  float total = 0.f;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) total += wsum[w];
  const float r = rsqrtf(total / float(P.N) + P.eps);
  auto norm_chunk = [&](int c, float (&sv)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) sv[i] *= r;
    *reinterpret_cast<uint4 *>(P.h_out + row + 8 * c) = pack8(sv);
  };
  if constexpr (CPT > 0) {
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int c = threadIdx.x + u * kThreads;
      if (c < chunks) norm_chunk(c, held[u]);
    }
  } else {
    // The thread's own chunks of x_out, written above by this same thread.
    for (int c = threadIdx.x; c < chunks; c += kThreads) {
      unpack8(*reinterpret_cast<const uint4 *>(P.x_out + row + 8 * c), held[0]);
      norm_chunk(c, held[0]);
    }
  }
}

}  // namespace
}  // namespace mcamd

using namespace mcamd;

extern "C" int mcamd_residual_rmsnorm(const void *x, const float *part, int64_t splits,
                                      const void *y, void *x_out, void *h_out, int64_t m,
                                      int64_t n, float eps, void *stream) {
  if (m < 0 || n <= 0 || n % 8 != 0 || m > (int64_t(1) << 31) - 1 || m * n >= (int64_t(1) << 40))
    return fail(MCAMD_EINVAL, "residual_rmsnorm: need m >= 0 and n > 0 a multiple of 8");
  if ((part == nullptr) == (y == nullptr))
    return fail(MCAMD_EINVAL, "residual_rmsnorm: pass the partials or y, not both");
  if (part && (splits < 1 || splits > 64))
    return fail(MCAMD_EINVAL, "residual_rmsnorm: splits must be in [1, 64]");
  if (!(eps >= 0.f)) return fail(MCAMD_EINVAL, "residual_rmsnorm: eps must be >= 0");
  if (m == 0) {
    clear_error();
    return MCAMD_OK;
  }
  if (!x || !x_out || !h_out) return fail(MCAMD_EINVAL, "residual_rmsnorm: null pointer");
  if (!aligned(x, 16) || !aligned(x_out, 16) || !aligned(h_out, 16) ||
      (part && !aligned(part, 16)) || (y && !aligned(y, 16)))
    return fail(MCAMD_EINVAL, "residual_rmsnorm: buffers must be 16-byte aligned");
  ResParams P;
  P.x = static_cast<const uint16_t *>(x);
  P.y = static_cast<const uint16_t *>(y);
  P.part = part;
  P.x_out = static_cast<uint16_t *>(x_out);
  P.h_out = static_cast<uint16_t *>(h_out);
  P.M = int(m);
  P.N = int(n);
  P.S = part ? int(splits) : 0;
  P.eps = eps;
  const int64_t chunks = n / 8;
  const dim3 grid{unsigned(m), 1, 1}, block{unsigned(kThreads), 1, 1};
  hipStream_t s = as_stream(stream);
  if (P.S > kMaxBatchedSplits && P.S <= 2 * kMaxBatchedSplits && chunks <= 2 * kThreads) {
    hipLaunchKernelGGL((residual_rmsnorm_kernel<2, 2 * kMaxBatchedSplits>), grid, block, 0, s, P.x, P.y, P.part, P.x_out, P.h_out, P.M, P.N, P.S, P.eps);
  } else if (P.S > kMaxBatchedSplits) {
    hipLaunchKernelGGL((residual_rmsnorm_kernel<0, 0>), grid, block, 0, s, P.x, P.y, P.part, P.x_out, P.h_out, P.M, P.N, P.S, P.eps);
  } else if (chunks <= kThreads) {
    hipLaunchKernelGGL((residual_rmsnorm_kernel<1, kMaxBatchedSplits>), grid, block, 0, s, P.x, P.y, P.part, P.x_out, P.h_out, P.M, P.N, P.S, P.eps);
  } else if (chunks <= 2 * kThreads) {
    hipLaunchKernelGGL((residual_rmsnorm_kernel<2, kMaxBatchedSplits>), grid, block, 0, s, P.x, P.y, P.part, P.x_out, P.h_out, P.M, P.N, P.S, P.eps);
  } else if (chunks <= 4 * kThreads) {
    hipLaunchKernelGGL((residual_rmsnorm_kernel<4, kMaxBatchedSplits>), grid, block, 0, s, P.x, P.y, P.part, P.x_out, P.h_out, P.M, P.N, P.S, P.eps);
  } else {
    hipLaunchKernelGGL((residual_rmsnorm_kernel<0, kMaxBatchedSplits>), grid, block, 0, s, P.x, P.y, P.part, P.x_out, P.h_out, P.M, P.N, P.S, P.eps);
  }
  return launch_status("residual_rmsnorm");
}
