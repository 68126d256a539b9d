// y = x . W^T for a decode-sized batch: x (M, K) bf16 with M <= 64 rows, W (N, K) bf16 (the
// nn.Linear weight layout), y (M, N) bf16, fp32 accumulation.
//
// Replaces F.linear in Linear.forward (modelcore/components/linear.py:13-14) when a decode step
// feeds at most 64 rows: every weight byte is then used at most 64 times, so the product is bound
// by reading W from HBM once -- cold, since a decode step walks through gigabytes of weights,
// far more than any cache holds.
//
// Work split. A workgroup owns 16 WAVES consecutive rows of W (outputs n) and a K-range
// [k0, k0 + K / S); wave w owns rows 16 w .. 16 w + 15 of the tile, and all waves share the
// activation rows. Two shapes: eight waves (128-row tiles) for more than 16 activation rows
// whenever the 128-row tiles times the K split fit one workgroup per CU (wide projections with
// S = 1, the others with S chosen for 128-row tiles), where sharing one activation tile among
// more weight rows halves the activation traffic; four waves (64-row tiles) with the K-range
// split S ways otherwise. With S > 1 the S partial products are summed by a second pass in a
// fixed order, so results never depend on timing (nor on the tile shape: a partial's k order is
// the same).
//
// Data path. The K-range is walked in stages of 128: one stage is 16 WAVES rows x 256 bytes of W
// and 64 rows x 256 bytes of x, brought into LDS by buffer_load ... lds (16 bytes per lane, four
// rows of 256 contiguous bytes per instruction, so every HBM line is read whole), RING - 1
// stages ahead in a ring of RING (4 with four waves, 3 with eight: 128 and 144 KB of LDS). Each
// wave moves its own 16 rows of W and a share of x. W is loaded non-temporal (read once: its
// lines should not push the activations out of L2). The buffer resources bound every read (rows
// of x past M read as zero). In LDS a row keeps its sixteen 16-byte chunks, chunk c of row r at
// slot c ^ (r % 16), so the fragment reads below -- sixteen rows, one chunk each -- fall on
// distinct banks.
//
// Products: v_mfma_f32_16x16x32_bf16 with A = 16 rows of W x 32 k (lane l: row l % 16, k 8 (l / 16)
// .. + 7), B = 32 k x 16 rows of x, MB blocks for M <= 16 MB; accumulators D[n][m] with lane l
// holding n = 4 (l / 16) + i, m = l % 16.
#include "kernels.h"

namespace mcamd {
namespace {

constexpr int KC = 128;              // k per stage
constexpr int kSteps = KC / 32;      // MFMA k-steps per stage
constexpr int kXRows = 64;           // activation rows staged (past M: zeros)
constexpr int kStageX = kXRows * KC; // elements of one x stage
constexpr int kNonTemporal = 2;      // buffer-load cache policy bits: nt

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct LinParams {
  const uint16_t *x, *w;
  uint16_t *y;
  float *part;  // [S][M][N] fp32 partials when S > 1 or raw
  int64_t ldx, ldy;
  int M, N, K, S;
  int raw;      // write the partials (fp32) even for S = 1, and leave the sum to the consumer
  int gated;    // W holds [gate; up] interleaved in 64-row blocks: write silu(gate) * up to y
  int w_tiled;  // W stored as (N / 64, K / 128, 64, 128) blocks instead of row-major (N, K)
};

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return uint32_t(uintptr_t((const __attribute__((address_space(3))) void *)(p)));
}
// LDS reads issued as inline asm: the compiler does not track them, so every use of a result sits
// behind wait_lgkm, an explicit `s_waitcnt lgkmcnt(N)` that takes the results as operands.
template <int OFF>
__device__ __forceinline__ void ds_read_b128(bf16x8 &d, uint32_t addr) {
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(d) : "v"(addr), "i"(OFF));
}
template <int N>
__device__ __forceinline__ void wait_lgkm(bf16x8 &a, bf16x8 &b0, bf16x8 &b1, bf16x8 &b2,
                                          bf16x8 &b3) {
  static_assert(N >= 0 && N <= 15, "lgkmcnt takes 0..15");
  asm volatile("s_waitcnt lgkmcnt(%5)"
               : "+v"(a), "+v"(b0), "+v"(b1), "+v"(b2), "+v"(b3)
               : "i"(N));
}
// wait_lgkm<n> for a count known only after unrolling (the branches fold away).
template <int N = 15>
__device__ __forceinline__ void wait_lgkm_n(int n, bf16x8 &a, bf16x8 &b0, bf16x8 &b1, bf16x8 &b2,
                                            bf16x8 &b3) {
  if (n == N)
    wait_lgkm<N>(a, b0, b1, b2, b3);
  else if constexpr (N > 0)
    wait_lgkm_n<N - 1>(n, a, b0, b1, b2, b3);
}
// s_waitcnt with vmcnt(N) and the other counters left alone (vmcnt's low 4 bits at 3:0, high
// 2 bits at 15:14).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt takes 0..63");
  __builtin_amdgcn_s_waitcnt((N & 15) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

__device__ __forceinline__ uint16_t to_bf16(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}
__device__ __forceinline__ float round_bf16(float x) { return __uint_as_float(uint32_t(to_bf16(x)) << 16); }

// h = silu(gate) * up as torch computes it on bf16 tensors: the product's outputs rounded to
// bf16, silu in fp32 rounded to bf16, the product in fp32 rounded to bf16.
__device__ __forceinline__ uint16_t silu_mul_bf16(float gate, float up) {
  const float g = round_bf16(gate), u = round_bf16(up);
  const float a = round_bf16(g / (1.f + expf(-g)));
  return to_bf16(a * u);
}

// The leading arguments repeat the fields of P that the tile set-up needs, so that they arrive
// preloaded in SGPRs at dispatch (the library is built with kernarg preloading, which covers
// scalar arguments only) rather than through a load from the kernel-argument buffer.
template <int WAVES, int MB>  // MB blocks of 16 activation rows: M <= 16 MB
__global__ __launch_bounds__(64 * WAVES, 1) void linear_skinny_kernel(
    const uint16_t *a_x, const uint16_t *a_w, int64_t a_ldx, int a_M, int a_N, int a_K, int a_S,
    int a_w_tiled, LinParams P) {
  P.x = a_x;
  P.w = a_w;
  P.ldx = a_ldx;
  P.M = a_M;
  P.N = a_N;
  P.K = a_K;
  P.S = a_S;
  P.w_tiled = a_w_tiled;
  constexpr int kRows = 16 * WAVES;         // rows of W per workgroup
  constexpr int kRing = WAVES == 8 ? 3 : 4; // LDS stages
  constexpr int kStageW = kRows * KC;       // elements of one W stage
  constexpr int kXPer = kXRows / 4 / WAVES; // x DMA instructions per wave and stage
  constexpr int kPer = 4 + kXPer;           // loads per wave and stage
  __shared__ __attribute__((aligned(1024))) uint16_t sW[kRing][kStageW];
  __shared__ __attribute__((aligned(1024))) uint16_t sX[kRing][kStageX];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n0 = blockIdx.x * kRows;
  const int ks = P.K / P.S;
  const int k_begin = blockIdx.y * ks;
  const int stages = ks / KC;

  const uint32_t wbytes = uint32_t(min(kRows, P.N - n0)) * uint32_t(P.K) * 2u;
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(P.w + int64_t(n0) * P.K), 0, int(wbytes), 0x00020000);
  const uint32_t xbytes = uint32_t(P.M) * uint32_t(P.ldx) * 2u;
  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc((void *)P.x, 0, int(xbytes), 0x00020000);

  // DMA: an instruction moves 4 rows (1 KB); lane i lands at LDS slot i % 16 of row i / 16 of
  // those four and reads the global chunk that belongs there. Wave w moves W rows 16 w .. 16 w
  // + 15 (four instructions) and x rows 4 (w + WAVES u) .. + 3 for u < kXPer.
  const int drow = lane >> 4;
  const int dslot = lane & 15;
  auto issue_stage = [&](int st, int buf) {
    const uint32_t kb = uint32_t(k_begin + st * KC) * 2u;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int r0 = 4 * (4 * wave + jj);
      const int r = r0 + drow;
      const uint32_t chunk = uint32_t(dslot ^ (r & 15));
      // Row-major: row r of the tile, bytes kb .. kb + 255. Tiled: the tile's 64-row group
      // r / 64 (K * 128 bytes each, at the same place as in row-major), its 16 KB block of this
      // stage, row r % 64 of the block -- an instruction reads 1 KB contiguous.
      const uint32_t wo = P.w_tiled ? uint32_t(r >> 6) * uint32_t(P.K) * 128u + kb * 64u +
                                          uint32_t(r & 63) * 256u + chunk * 16u
                                    : uint32_t(r) * uint32_t(P.K) * 2u + kb + chunk * 16u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rw, (__attribute__((address_space(3))) void *)(&sW[buf][r0 * KC]), 16, int(wo), 0, 0,
          kNonTemporal);
    }
#pragma unroll
    for (int u = 0; u < kXPer; ++u) {
      const int r0 = 4 * (wave + WAVES * u);
      const int r = r0 + drow;
      const uint32_t chunk = uint32_t(dslot ^ (r & 15));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rx, (__attribute__((address_space(3))) void *)(&sX[buf][r0 * KC]), 16,
          int(uint32_t(r) * uint32_t(P.ldx) * 2u + kb + chunk * 16u), 0, 0, 0);
    }
  };

  f32x4 acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int fr = lane & 15;  // fragment row (W row within the wave's 16, or x row in a block)
  const int fq = lane >> 4;  // which 8 k of the 32
  const int wr = 16 * wave + fr;

  // LDS byte addresses of this lane's fragments in buffer 0: k-step s reads chunk 4 s + fq of
  // W row wr and of x row fr (x row 16 mb + fr is mb * 16 rows further, an immediate offset);
  // both rows have r % 16 == fr, so the chunk sits at slot (4 s + fq) ^ fr.
  uint32_t a_at[kSteps], b_at[kSteps];
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const uint32_t slot = uint32_t(((4 * s + fq) ^ fr) << 4);
    a_at[s] = lds_addr(&sW[0][0]) + uint32_t(wr * KC * 2) + slot;
    b_at[s] = lds_addr(&sX[0][0]) + uint32_t(fr * KC * 2) + slot;
  }
  bf16x8 a[kSteps], b[kSteps][4];
#pragma unroll
  for (int s = 0; s < kSteps; ++s)
#pragma unroll
    for (int mb = MB; mb < 4; ++mb) b[s][mb] = bf16x8{};

  // Stages 0 .. kRing - 2 before the loop; stage st + kRing - 1 goes into buffer
  // (st + kRing - 1) % kRing, last read in iteration st - 1, after the barrier of iteration st.
  // A stage is published by each wave's own vmcnt wait (an LDS DMA is counted until its data is
  // in LDS) followed by a bare s_barrier: __syncthreads' fence would make the compiler wait for
  // every load in flight, draining the prefetch at each stage. The asm fragment reads keep their
  // place on either side of the barrier (both have side effects), and they are complete
  // (wait_lgkm) before the barrier that lets a later stage overwrite their buffer.
#pragma unroll
  for (int st = 0; st < kRing - 1; ++st)
    if (st < stages) issue_stage(st, st);
  for (int st = 0; st < stages; ++st) {
    const int ahead = min(stages - 1 - st, kRing - 2);  // younger stages that may stay pending
    if (ahead >= 2)
      wait_vm<2 * kPer>();
    else if (ahead == 1)
      wait_vm<kPer>();
    else
      wait_vm<0>();
    __builtin_amdgcn_s_barrier();
    if (st + kRing - 1 < stages) issue_stage(st + kRing - 1, (st + kRing - 1) % kRing);
    const uint32_t bw = uint32_t(st % kRing) * uint32_t(kStageW * 2);
    const uint32_t bx = uint32_t(st % kRing) * uint32_t(kStageX * 2);
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      ds_read_b128<0>(a[s], a_at[s] + bw);
      ds_read_b128<0>(b[s][0], b_at[s] + bx);
      if constexpr (MB > 1) ds_read_b128<16 * KC * 2>(b[s][1], b_at[s] + bx);
      if constexpr (MB > 2) ds_read_b128<32 * KC * 2>(b[s][2], b_at[s] + bx);
      if constexpr (MB > 3) ds_read_b128<48 * KC * 2>(b[s][3], b_at[s] + bx);
    }
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      wait_lgkm_n((kSteps - 1 - s) * (1 + MB), a[s], b[s][0], b[s][1], b[s][2], b[s][3]);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[s], b[s][mb], acc[mb], 0, 0, 0);
    }
  }

  // acc[mb][i] = y[m = 16 mb + l % 16][n = n0 + 16 w + 4 (l / 16) + i].
  if constexpr (WAVES == 8) {
    if (P.gated) {
      // Rows 0..63 of the tile are gate rows j, rows 64..127 the up rows of the same j: wave
      // w + 4 holds, lane for lane, the up values of wave w's gate values. They pass through
      // LDS (the W ring, free once every wave is past its last stage: a full __syncthreads, so
      // that no store below can be moved above it).
      float *xch = reinterpret_cast<float *>(&sW[0][0]);
      __syncthreads();
      if (wave >= 4) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int i = 0; i < 4; ++i) xch[(((wave - 4) * MB + mb) * 4 + i) * 64 + lane] = acc[mb][i];
      }
      __syncthreads();
      if (wave >= 4) return;
      const int j = blockIdx.x * 64 + 16 * wave + 4 * fq;  // hidden unit of acc[.][0]
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const int m = 16 * mb + fr;
        if (m >= P.M) continue;
        uint16_t hv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          hv[i] = silu_mul_bf16(acc[mb][i], xch[((wave * MB + mb) * 4 + i) * 64 + lane]);
        *reinterpret_cast<uint2 *>(P.y + int64_t(m) * P.ldy + j) =
            uint2{uint32_t(hv[0]) | (uint32_t(hv[1]) << 16), uint32_t(hv[2]) | (uint32_t(hv[3]) << 16)};
      }
      return;
    }
  }
  const int n = n0 + 16 * wave + 4 * fq;
  if (n >= P.N) return;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = 16 * mb + fr;
    if (m >= P.M) continue;
    if (P.S == 1 && !P.raw) {
      const uint32_t lo = uint32_t(to_bf16(acc[mb][0])) | (uint32_t(to_bf16(acc[mb][1])) << 16);
      const uint32_t hi = uint32_t(to_bf16(acc[mb][2])) | (uint32_t(to_bf16(acc[mb][3])) << 16);
      *reinterpret_cast<uint2 *>(P.y + int64_t(m) * P.ldy + n) = uint2{lo, hi};
    } else {
      *reinterpret_cast<f32x4 *>(P.part + (int64_t(blockIdx.y) * P.M + m) * P.N + n) = acc[mb];
    }
  }
}

// y[m][n] = sum over the S partials in order, four n per thread.
__global__ __launch_bounds__(256) void linear_reduce_kernel(LinParams P) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;  // float4 index
  const int64_t per_row = P.N / 4;
  if (i >= int64_t(P.M) * per_row) return;
  const int64_t m = i / per_row, n = (i - m * per_row) * 4;
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
  for (int k = 0; k < P.S; ++k)
    s += *reinterpret_cast<const f32x4 *>(P.part + (int64_t(k) * P.M + m) * P.N + n);
  const uint32_t lo = uint32_t(to_bf16(s[0])) | (uint32_t(to_bf16(s[1])) << 16);
  const uint32_t hi = uint32_t(to_bf16(s[2])) | (uint32_t(to_bf16(s[3])) << 16);
  *reinterpret_cast<uint2 *>(P.y + m * P.ldy + n) = uint2{lo, hi};
}

template <int WAVES>
void launch_skinny(const LinParams &P, hipStream_t s) {
  const dim3 grid(unsigned((P.N + 16 * WAVES - 1) / (16 * WAVES)), unsigned(P.S));
  const dim3 block(64 * WAVES);
  if (P.M <= 16)
    hipLaunchKernelGGL((linear_skinny_kernel<WAVES, 1>), grid, block, 0, s, P.x, P.w, P.ldx, P.M, P.N, P.K, P.S, P.w_tiled, P);
  else if (P.M <= 32)
    hipLaunchKernelGGL((linear_skinny_kernel<WAVES, 2>), grid, block, 0, s, P.x, P.w, P.ldx, P.M, P.N, P.K, P.S, P.w_tiled, P);
  else if (P.M <= 48)
    hipLaunchKernelGGL((linear_skinny_kernel<WAVES, 3>), grid, block, 0, s, P.x, P.w, P.ldx, P.M, P.N, P.K, P.S, P.w_tiled, P);
  else
    hipLaunchKernelGGL((linear_skinny_kernel<WAVES, 4>), grid, block, 0, s, P.x, P.w, P.ldx, P.M, P.N, P.K, P.S, P.w_tiled, P);
}

}  // namespace
}  // namespace mcamd

using namespace mcamd;

extern "C" size_t mcamd_linear_bf16_workspace_bytes(int64_t m, int64_t n, int64_t k_splits) {
  return k_splits > 1 ? size_t(k_splits) * size_t(m) * size_t(n) * sizeof(float) : 0;
}

namespace {

// Argument checks shared by the two entry points; fills P on success.
int check_linear(const void *x, int64_t ldx, const void *w, int64_t m, int64_t n, int64_t k,
                 int64_t k_splits, LinParams &P) {
  if (m < 0 || m > 64)
    return fail(MCAMD_EUNSUPPORTED, "linear_bf16: m must be at most 64 (decode-sized batches)");
  if (k_splits < 1 || k_splits > 64)
    return fail(MCAMD_EINVAL, "linear_bf16: k_splits must be in [1, 64]");
  if (n <= 0 || k <= 0 || n % 64 != 0 || k % (KC * k_splits) != 0)
    return fail(MCAMD_EUNSUPPORTED,
                "linear_bf16: n must be a multiple of 64 and k of 128 * k_splits");
  if (n > (int64_t(1) << 30) || int64_t(128) * k * 2 >= (int64_t(1) << 31))
    return fail(MCAMD_EUNSUPPORTED, "linear_bf16: n or k too large");
  if (m > 0) {
    if (!x || !w) return fail(MCAMD_EINVAL, "linear_bf16: null pointer");
    if (ldx < k || ldx % 8 != 0)
      return fail(MCAMD_EINVAL, "linear_bf16: need ldx >= k, a multiple of 8");
    if (kXRows * ldx * 2 >= (int64_t(1) << 31))
      return fail(MCAMD_EUNSUPPORTED, "linear_bf16: activations too large");
    if (!aligned(x, 16) || !aligned(w, 16))
      return fail(MCAMD_EINVAL, "linear_bf16: x and w must be 16-byte aligned");
  }
  P = LinParams{};
  P.x = static_cast<const uint16_t *>(x);
  P.w = static_cast<const uint16_t *>(w);
  P.ldx = ldx;
  P.M = int(m);
  P.N = int(n);
  P.K = int(k);
  P.S = int(k_splits);
  return MCAMD_OK;
}

void launch_linear(const LinParams &P, hipStream_t s) {
  // Eight waves where the activation tile is large enough for its traffic to matter and the
  // 128-row tiles (times the K split) fit one workgroup per CU (measured on MI355X, cold weights,
  // 28672 x 4096: 64 rows 49.2 us against 57.6 with four waves; 16 rows 49.2 against 47.3; with
  // 64 rows, 6144 x 4096 at S = 4 12.6 us against 14.4 for 64-row tiles at S = 2, 4096 x 14336
  // at S = 8 22.8 against 25.1 at S = 4); four waves otherwise.
  const bool wide = P.S == 1 && P.N >= 192 * 128;
  const bool split128 = P.S > 1 && P.N % 128 == 0 && int64_t(P.N / 128) * P.S <= 256;
  if (P.M > 16 && (wide || split128))
    launch_skinny<8>(P, s);
  else
    launch_skinny<4>(P, s);
}

}  // namespace

extern "C" int mcamd_linear_bf16(const void *x, int64_t ldx, const void *w, void *y, int64_t ldy,
                                 int64_t m, int64_t n, int64_t k, int64_t k_splits,
                                 void *workspace, size_t workspace_bytes, void *stream) {
  LinParams P;
  int st = check_linear(x, ldx, w, m, n, k, k_splits, P);
  if (st != MCAMD_OK) return st;
  if (m == 0) {
    clear_error();
    return MCAMD_OK;
  }
  if (!y) return fail(MCAMD_EINVAL, "linear_bf16: null pointer");
  if (ldy < n || ldy % 4 != 0 || !aligned(y, 8))
    return fail(MCAMD_EINVAL, "linear_bf16: need ldy >= n (a multiple of 4), y 8-byte aligned");
  if (k_splits > 1 &&
      (!workspace || workspace_bytes < mcamd_linear_bf16_workspace_bytes(m, n, k_splits) ||
       !aligned(workspace, 16)))
    return fail(MCAMD_EWORKSPACE, "linear_bf16: workspace missing or too small for k_splits");
  P.y = static_cast<uint16_t *>(y);
  P.ldy = ldy;
  P.part = static_cast<float *>(workspace);
  hipStream_t s = as_stream(stream);
  launch_linear(P, s);
  st = launch_status("linear_bf16");
  if (st != MCAMD_OK || k_splits == 1) return st;
  const int64_t quads = m * (n / 4);
  hipLaunchKernelGGL(linear_reduce_kernel, dim3(unsigned((quads + 255) / 256)), dim3(256), 0, s,
                     P);
  return launch_status("linear_bf16 reduce");
}

extern "C" int mcamd_linear_bf16_gated(const void *x, int64_t ldx, const void *w, void *h,
                                       int64_t ldh, int64_t m, int64_t hidden, int64_t k, int act,
                                       int w_tiled, void *stream) {
  if (act != MCAMD_ACT_SILU)
    return fail(MCAMD_EUNSUPPORTED, "linear_bf16_gated: only silu is supported");
  if (hidden <= 0 || hidden % 64 != 0)
    return fail(MCAMD_EUNSUPPORTED, "linear_bf16_gated: hidden must be a multiple of 64");
  LinParams P;
  int st = check_linear(x, ldx, w, m, 2 * hidden, k, 1, P);
  if (st != MCAMD_OK) return st;
  if (m == 0) {
    clear_error();
    return MCAMD_OK;
  }
  if (!h || ldh < hidden || ldh % 4 != 0 || !aligned(h, 8))
    return fail(MCAMD_EINVAL, "linear_bf16_gated: need h with ldh >= hidden (a multiple of 4)");
  P.y = static_cast<uint16_t *>(h);
  P.ldy = ldh;
  P.gated = 1;
  P.w_tiled = w_tiled != 0;
  launch_skinny<8>(P, as_stream(stream));  // a 128-row tile holds 64 gate and their 64 up rows
  return launch_status("linear_bf16_gated");
}

extern "C" int mcamd_linear_bf16_partials(const void *x, int64_t ldx, const void *w, float *part,
                                          int64_t m, int64_t n, int64_t k, int64_t k_splits,
                                          void *stream) {
  LinParams P;
  int st = check_linear(x, ldx, w, m, n, k, k_splits, P);
  if (st != MCAMD_OK) return st;
  if (m == 0) {
    clear_error();
    return MCAMD_OK;
  }
  if (!part || !aligned(part, 16))
    return fail(MCAMD_EINVAL, "linear_bf16_partials: part must be a 16-byte aligned buffer");
  P.part = part;
  P.raw = 1;
  launch_linear(P, as_stream(stream));
  return launch_status("linear_bf16_partials");
}
