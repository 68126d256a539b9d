// y = x . W^T for a decode-sized batch: x (M, K) bf16 with M <= 64 rows, W (N, K) bf16 (the
// nn.Linear weight layout), y (M, N) bf16, fp32 accumulation.
//
// Replaces F.linear in Linear.forward (modelcore/components/linear.py:13-14) when a decode step
// feeds at most 64 rows: there every weight byte is used M times, so the product is bound by
// reading W from HBM once, and a library GEMM tiled for large M leaves much of that bandwidth
// unused on these shapes.
//
// Work split. A workgroup of eight waves owns RB * 32 consecutive rows of W (outputs n) and the
// whole K; wave w takes the K-slice [w K / 8, (w + 1) K / 8). Per 16-wide k-step a wave loads RB
// fragments of W (32 rows x 16 k, 16 bytes per lane) and MB fragments of x (32 rows x 16 k) and
// runs RB * MB v_mfma_f32_32x32x16_bf16 with W as the A operand and x as the B operand, so the
// accumulators hold y^T blocks: n = 8 (r / 4) + 4 h + r % 4 of the block, m = lane % 32. The
// eight K-slice partials meet in LDS (padded so neither the writes nor the reads collide in
// banks) and are summed in a fixed order -- the result does not depend on timing -- then written
// as bf16 with consecutive lanes on consecutive n. Rows m >= M of x read as zero.
//
// Loads are issued one group of U (4 or 8) k-steps ahead of the products that use them, into the
// registers of a second buffer, so each wave keeps 4-8 KiB of W in flight.
#include "kernels.h"

namespace mcamd {
namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

struct LinParams {
  const uint16_t *x, *w;
  uint16_t *y;
  int64_t ldx, ldy;
  int M, N, K;
};

__device__ __forceinline__ f32x16 mfma(const bf16x8 &a, const bf16x8 &b, const f32x16 &c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 load16(const uint16_t *p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(p));
}

__device__ __forceinline__ uint16_t to_bf16(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

template <int RB, int MB, int U>
__global__ __launch_bounds__(kThreads, 1) void linear_skinny_kernel(LinParams P) {
  constexpr int NR = RB * 32;      // rows of W (outputs n) per workgroup
  constexpr int MP = MB * 32 + 1;  // padded m stride of the LDS partials
  __shared__ float part[kWaves * NR * MP];  // [wave][n][m]

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int h = lane >> 5;
  const int col = lane & 31;
  const int n0 = blockIdx.x * NR;
  const int ks = P.K / kWaves;  // this wave's K-slice, a multiple of 16 * U
  const int k_begin = wave * ks;
  const int steps = ks / 16;

  const uint16_t *wrow[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
    wrow[rb] = P.w + int64_t(n0 + rb * 32 + col) * P.K + k_begin + 8 * h;
  const uint16_t *xrow[MB];
  bool xlive[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = mb * 32 + col;
    xlive[mb] = m < P.M;
    xrow[mb] = P.x + int64_t(xlive[mb] ? m : 0) * P.ldx + k_begin + 8 * h;
  }

  f32x16 acc[RB][MB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[rb][mb][e] = 0.f;

  const bf16x8 zero8 = {};
  bf16x8 wa[2][U][RB], xb[2][U][MB];
  auto load_group = [&](int buf, int s0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int off = 16 * (s0 + u);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) wa[buf][u][rb] = load16(wrow[rb] + off);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        // Unconditional load (dead rows read row 0), then a select: no branch between the
        // loads, so the waits before the products count them exactly.
        const bf16x8 v = load16(xrow[mb] + off);
        xb[buf][u][mb] = xlive[mb] ? v : zero8;
      }
    }
  };
  auto mul_group = [&](int buf) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          acc[rb][mb] = mfma(wa[buf][u][rb], xb[buf][u][mb], acc[rb][mb]);
  };

  load_group(0, 0);
  int g = 0;
  for (; g + U < steps; g += 2 * U) {
    load_group(1, g + U);
    mul_group(0);
    // Unconditional (the last pass reloads a group it already has), so the waits before the
    // products count the loads exactly.
    load_group(0, min(g + 2 * U, steps - U));
    mul_group(1);
  }
  if (g < steps) mul_group(0);

  // Partials into LDS: part[wave][n][m], m contiguous (lanes of a half write consecutive m).
  float *mine = part + wave * NR * MP;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int n = rb * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        mine[n * MP + mb * 32 + col] = acc[rb][mb][r];
      }
  __syncthreads();
  // Sum the eight K-slices in wave order; consecutive threads take consecutive n.
  for (int i = threadIdx.x; i < NR * MB * 32; i += kThreads) {
    const int n = i % NR;
    const int m = i / NR;
    if (m >= P.M) break;
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) s += part[(w * NR + n) * MP + m];
    P.y[int64_t(m) * P.ldy + n0 + n] = to_bf16(s);
  }
}

template <int RB, int MB>
void launch(const LinParams &P, hipStream_t stream) {
  // Eight k-steps per load group where the K-slices allow it (twice the bytes in flight), else
  // four; 64-row groups with two x blocks keep four (eight would spill).
  const dim3 grid(unsigned(P.N / (RB * 32)));
  if constexpr (RB == 2 && MB == 2) {
    hipLaunchKernelGGL((linear_skinny_kernel<RB, MB, 4>), grid, dim3(kThreads), 0, stream, P);
  } else {
    if (P.K % (16 * 8 * kWaves) == 0)
      hipLaunchKernelGGL((linear_skinny_kernel<RB, MB, 8>), grid, dim3(kThreads), 0, stream, P);
    else
      hipLaunchKernelGGL((linear_skinny_kernel<RB, MB, 4>), grid, dim3(kThreads), 0, stream, P);
  }
}

}  // namespace
}  // namespace mcamd

using namespace mcamd;

extern "C" int mcamd_linear_bf16(const void *x, int64_t ldx, const void *w, void *y, int64_t ldy,
                                 int64_t m, int64_t n, int64_t k, int rows_per_group,
                                 void *stream) {
  if (m < 0 || m > 64)
    return fail(MCAMD_EUNSUPPORTED, "linear_bf16: m must be at most 64 (decode-sized batches)");
  if (n <= 0 || k <= 0 || n % 32 != 0 || k % (16 * 4 * kWaves) != 0)
    return fail(MCAMD_EUNSUPPORTED, "linear_bf16: n must be a multiple of 32 and k of 512");
  if (n > (int64_t(1) << 30) || k > (int64_t(1) << 30))
    return fail(MCAMD_EUNSUPPORTED, "linear_bf16: n or k too large");
  if (rows_per_group != 32 && rows_per_group != 64)
    return fail(MCAMD_EINVAL, "linear_bf16: rows_per_group must be 32 or 64");
  if (rows_per_group == 64 && n % 64 != 0)
    return fail(MCAMD_EINVAL, "linear_bf16: rows_per_group 64 needs n a multiple of 64");
  if (m == 0) {
    clear_error();
    return MCAMD_OK;
  }
  if (!x || !w || !y) return fail(MCAMD_EINVAL, "linear_bf16: null pointer");
  if (ldx < k || ldy < n) return fail(MCAMD_EINVAL, "linear_bf16: ldx < k or ldy < n");
  if (!aligned(x, 16) || !aligned(w, 16) || ldx % 8 != 0)
    return fail(MCAMD_EINVAL, "linear_bf16: x and w must be 16-byte aligned, ldx a multiple of 8");
  LinParams P;
  P.x = static_cast<const uint16_t *>(x);
  P.w = static_cast<const uint16_t *>(w);
  P.y = static_cast<uint16_t *>(y);
  P.ldx = ldx;
  P.ldy = ldy;
  P.M = int(m);
  P.N = int(n);
  P.K = int(k);
  hipStream_t s = as_stream(stream);
  if (rows_per_group == 64) {
    if (m > 32)
      launch<2, 2>(P, s);
    else
      launch<2, 1>(P, s);
  } else {
    if (m > 32)
      launch<1, 2>(P, s);
    else
      launch<1, 1>(P, s);
  }
  return launch_status("linear_bf16");
}
