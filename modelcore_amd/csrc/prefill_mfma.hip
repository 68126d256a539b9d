// Chunked-prefill attention against the cache prefix on the bf16 matrix cores (gfx950), for bf16
// caches with head_dim 128.
//
// Semantics: modelcore/kernels/flash_attn.py:226-244 (uniform rows: explicit causal + window mask
// with row offset Tk - Tq) and :362-364 (ragged rows). Query t of row b sits at
// p = cache_seqlens[b] + t and attends keys col <= p with p - col <= window when window >= 0;
// query head h reads KV head h / G; scale 1/sqrt(128). The append has already run, so the
// prefix includes the chunk itself.
//
// Work split. A workgroup owns one (row b, KV head) and 256 (position, query head) pairs of it:
// QT = 256 / G consecutive positions times the G query heads that share the KV head, head
// fastest (so one position's G heads are one contiguous run of q). Every K/V tile staged in LDS
// therefore serves the whole GQA group. Workgroup ids put the query tiles of one (b, KV head)
// 8 * k ids apart, so they land on the same XCD and share its L2.
//
// Each of the four waves owns 64 pairs (two 32-wide column blocks) and computes, per tile of 64
// keys, with v_mfma_f32_32x32x16_bf16:
//   S^T (keys x pairs) = K (keys x D) . Q^T (D x pairs)       A = K from LDS, B = Q in registers
//   O^T (D x pairs)   += V^T (D x keys) . P^T (keys x pairs)   A = V^T via ds_read_tr16_b64
// Computing the transposed scores makes the score accumulators come out with one pair per lane
// (lane l holds pair l % 32 of the block, keys 8j + 4(l/32) + i), which is the layout the second
// product wants for its B operand: the eight consecutive accumulators of a 16-key step are that
// step's B fragment, once packed to bf16. The 16 keys of a step are taken in the order the
// accumulators hold them (4h..4h+3, then 8+4h..8+4h+3 for lane half h); the V^T fragment reads the
// same keys, as two LDS transpose reads of four rows each.
//
// Online softmax per pair in fp32 (exp2 domain): the running maximum is raised only when a tile's
// maximum exceeds it by more than 2^8, so most tiles skip the rescale of O. Tiles entirely inside
// every pair's visible range skip the masking.
//
// LDS: two buffers of one K and one V tile (64 rows of 256 bytes each), filled straight from
// HBM by global_load_lds_dwordx4 (no registers involved) while the other buffer is computed on.
// Each 16-byte chunk c of row r sits at slot c ^ g(r), a swizzle under which the 16-byte K reads
// (32 consecutive rows, one chunk) and the 8-byte transpose reads of V (4 consecutive rows, two
// chunks) fall into distinct banks.
#include "kernels.h"

#include <cmath>

namespace mcamd {
namespace {

constexpr int D = 128;
constexpr int kPairs = 256;        // (position, head) pairs per workgroup
constexpr int KT = 64;             // keys per tile
constexpr int TILE = KT * D;       // elements of one K (or V) tile in LDS
constexpr float kRescaleSlack = 8.f;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 lds_bf16x4 __attribute__((__vector_size__(4 * sizeof(__bf16))));

struct MfmaParams {
  const uint16_t *q, *k_cache, *v_cache;
  const int32_t *seqlens;
  uint16_t *out;
  int T_new, H, H_kv, G, QT, T_max, window, n_bh;
  int64_t cache_b;
  float scale_log2;
};

__device__ __forceinline__ f32x16 mfma(const bf16x8 &a, const bf16x8 &b, const f32x16 &c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Four consecutive LDS rows of one column, transposed into a lane: lane L of each 16-lane group
// passes the address of row L / 4, columns 4 (L % 4) .. + 3 of a 4 x 16 block and receives
// column L of it.
__device__ __forceinline__ bf16x4 lds_read_tr(const uint16_t *p) {
  auto lp = (__attribute__((address_space(3))) lds_bf16x4 *)(p);
  return __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(lp));
}

// Swizzle of the 16-byte chunks of LDS row r (0..63): chunk c is stored at slot c ^ swz(r).
__device__ __forceinline__ int swz(int r) {
  return ((r & 3) << 1) | ((r >> 2) & 1) | (((r >> 3) & 1) << 3);
}

__device__ __forceinline__ void dma16(const uint16_t *src, uint16_t *lds_wave_base) {
  __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1))) *)(src),
                                   (void __attribute__((address_space(3))) *)(lds_wave_base), 16,
                                   0, 0);
}

__device__ __forceinline__ float exp2_or_zero(float x) {
  return x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(x);
}

__global__ __launch_bounds__(256, 1) void prefill_mfma_kernel(MfmaParams P) {
  __shared__ __attribute__((aligned(1024))) uint16_t sK[2][TILE];
  __shared__ __attribute__((aligned(1024))) uint16_t sV[2][TILE];

  const int bh = blockIdx.x % P.n_bh;
  const int qt = blockIdx.x / P.n_bh;
  const int b = bh / P.H_kv;
  const int kvh = bh - b * P.H_kv;
  const int q0 = qt * P.QT;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int h = lane >> 5;      // lane half
  const int col = lane & 31;    // pair within a 32-wide block

  const int s0 = P.seqlens[b];
  const int q_end = min(q0 + P.QT, P.T_new);  // positions [q0, q_end) of the chunk
  const bool row_ok = s0 >= 0 && int64_t(s0) + P.T_new <= P.T_max;

  // This lane's two pairs (one per 32-wide block).
  int pos[2], head[2];
  bool live[2];
#pragma unroll
  for (int nq = 0; nq < 2; ++nq) {
    const int pr = wave * 64 + nq * 32 + col;
    const int t = q0 + pr / P.G;
    live[nq] = pr < P.QT * P.G && t < q_end;
    pos[nq] = live[nq] ? t : q0;  // dead pairs compute on a live position, write nothing
    head[nq] = live[nq] ? pr - (pr / P.G) * P.G : 0;
  }
  auto out_at = [&](int nq) {
    return P.out + ((int64_t(b) * P.T_new + pos[nq]) * P.H + int64_t(kvh) * P.G + head[nq]) * D;
  };
  if (!row_ok) {
#pragma unroll
    for (int nq = 0; nq < 2; ++nq)
      if (live[nq])
        for (int d = h * 64; d < h * 64 + 64; ++d) out_at(nq)[d] = 0x7fc0;
    return;
  }

  // Q^T fragments: B[k = dim][n = pair], lane holds pair `col`, dims 16 kd + 8 h .. + 7.
  bf16x8 qf[2][8];
#pragma unroll
  for (int nq = 0; nq < 2; ++nq) {
    const uint16_t *qp = P.q + ((int64_t(b) * P.T_new + pos[nq]) * P.H + int64_t(kvh) * P.G + head[nq]) * D + 8 * h;
#pragma unroll
    for (int kd = 0; kd < 8; ++kd)
      qf[nq][kd] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(qp + 16 * kd));
  }
  int p_abs[2];
#pragma unroll
  for (int nq = 0; nq < 2; ++nq) p_abs[nq] = s0 + pos[nq];

  const int p_first = s0 + q0;
  const int p_last = s0 + q_end - 1;
  const int lo = P.window >= 0 ? max(0, p_first - P.window) : 0;
  const int hi = p_last;

  const int64_t tok = int64_t(P.H_kv) * D;
  const uint16_t *kbase = P.k_cache + int64_t(b) * P.cache_b + int64_t(kvh) * D;
  const uint16_t *vbase = P.v_cache + int64_t(b) * P.cache_b + int64_t(kvh) * D;

  // One tile = 64 rows x 16 chunks of 16 bytes per K and V. Wave w fills rows 16 w .. 16 w + 15
  // with four DMA instructions each (one instruction = 64 lanes x 16 bytes = 4 rows); lane i of
  // an instruction lands at slot i % 16 of row i / 16, so it fetches chunk slot ^ swz(row).
  const int dma_row = lane >> 4;
  const int dma_slot = lane & 15;
  auto issue_tile = [&](int k0, int buf) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = 16 * wave + 4 * j + dma_row;
      const int key = min(k0 + r, hi);
      const int c = dma_slot ^ swz(r);
      dma16(kbase + int64_t(key) * tok + c * 8, &sK[buf][(16 * wave + 4 * j) * D]);
      dma16(vbase + int64_t(key) * tok + c * 8, &sV[buf][(16 * wave + 4 * j) * D]);
    }
  };

  f32x16 o[4][2];
#pragma unroll
  for (int md = 0; md < 4; ++md)
#pragma unroll
    for (int nq = 0; nq < 2; ++nq)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[md][nq][e] = 0.f;
  float m[2] = {-INFINITY, -INFINITY};
  float l[2] = {0.f, 0.f};

  const int L16 = lane & 15;
  const int tr_row = L16 >> 2;
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (L16 & 3);

  issue_tile(lo, 0);
  int buf = 0;
  for (int k0 = lo; k0 <= hi; k0 += KT, buf ^= 1) {
    // This wave's DMA of the tile has landed; after the barrier every wave's has, and every wave
    // is done with the other buffer, which the next tile's DMA then refills.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    if (k0 + KT <= hi) issue_tile(k0 + KT, buf ^ 1);
    const uint16_t *tK = sK[buf];
    const uint16_t *tV = sV[buf];

    // S^T = K . Q^T over the tile: s[mk][nq][4j + i] is key 32 mk + 8 j + 4 h + i, pair `col`.
    f32x16 s[2][2];
#pragma unroll
    for (int mk = 0; mk < 2; ++mk)
#pragma unroll
      for (int nq = 0; nq < 2; ++nq)
#pragma unroll
        for (int e = 0; e < 16; ++e) s[mk][nq][e] = 0.f;
#pragma unroll
    for (int kd = 0; kd < 8; ++kd) {
#pragma unroll
      for (int mk = 0; mk < 2; ++mk) {
        const int r = 32 * mk + col;
        const bf16x8 a = __builtin_bit_cast(
            bf16x8, *reinterpret_cast<const uint4 *>(&tK[r * D + ((2 * kd + h) ^ swz(r)) * 8]));
#pragma unroll
        for (int nq = 0; nq < 2; ++nq) s[mk][nq] = mfma(a, qf[nq][kd], s[mk][nq]);
      }
    }

    // Mask the keys a pair may not see (tiles that straddle the diagonal or the window edge).
    const bool need_mask = (k0 + KT - 1 > p_first) || (P.window >= 0 && k0 < p_last - P.window);
    if (need_mask) {
#pragma unroll
      for (int mk = 0; mk < 2; ++mk)
#pragma unroll
        for (int nq = 0; nq < 2; ++nq)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int key = k0 + 32 * mk + 8 * (e >> 2) + 4 * h + (e & 3);
            const int dpos = p_abs[nq] - key;
            const bool ok = dpos >= 0 && (P.window < 0 || dpos <= P.window);
            if (!ok) s[mk][nq][e] = -INFINITY;
          }
    }

    // Online softmax per pair; the pair's 64 keys sit in this lane and its partner lane ^ 32.
    float mx[2];
#pragma unroll
    for (int nq = 0; nq < 2; ++nq) {
      float v = -INFINITY;
#pragma unroll
      for (int mk = 0; mk < 2; ++mk)
#pragma unroll
        for (int e = 0; e < 16; ++e) v = fmaxf(v, s[mk][nq][e]);
      v = fmaxf(v, __shfl_xor(v, 32, 64));
      mx[nq] = v * P.scale_log2;
    }
    const bool raise = (mx[0] > m[0] + kRescaleSlack) || (mx[1] > m[1] + kRescaleSlack);
    if (__builtin_amdgcn_ballot_w64(raise) != 0) {
#pragma unroll
      for (int nq = 0; nq < 2; ++nq) {
        const float m_new = fmaxf(m[nq], mx[nq]);
        const float alpha = m_new == -INFINITY ? 1.f : exp2_or_zero(m[nq] - m_new);
        l[nq] *= alpha;
#pragma unroll
        for (int md = 0; md < 4; ++md)
#pragma unroll
          for (int e = 0; e < 16; ++e) o[md][nq][e] *= alpha;
        m[nq] = m_new;
      }
    }
    bf16x8 pk[2][4];  // P^T fragments per (pair block, 16-key step)
#pragma unroll
    for (int nq = 0; nq < 2; ++nq) {
      const float m_use = m[nq] == -INFINITY ? 0.f : m[nq];
#pragma unroll
      for (int mk = 0; mk < 2; ++mk) {
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
          f32x8 pv;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float x = s[mk][nq][8 * sub + e];
            const float pe = __builtin_amdgcn_exp2f(fmaf(x, P.scale_log2, -m_use));
            pv[e] = pe;
            l[nq] += pe;
          }
          pk[nq][2 * mk + sub] = __builtin_convertvector(pv, bf16x8);
        }
      }
    }

    // O^T += V^T . P^T, 16 keys per step in the accumulators' order.
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int kb = 32 * (ks >> 1) + 16 * (ks & 1) + 4 * h;
#pragma unroll
      for (int md = 0; md < 4; ++md) {
        const int cc = 32 * md + tr_col;  // column this lane addresses
        const int r0 = kb + tr_row, r1 = r0 + 8;
        const bf16x4 lo4 = lds_read_tr(&tV[r0 * D + (((cc >> 3) ^ swz(r0)) << 3) + (cc & 7)]);
        const bf16x4 hi4 = lds_read_tr(&tV[r1 * D + (((cc >> 3) ^ swz(r1)) << 3) + (cc & 7)]);
        const bf16x8 a = __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
        for (int nq = 0; nq < 2; ++nq) o[md][nq] = mfma(a, pk[nq][ks], o[md][nq]);
      }
    }
  }

  // Normalise and write: o[md][nq][4j + i] is dim 32 md + 8 j + 4 h + i of pair `col`.
#pragma unroll
  for (int nq = 0; nq < 2; ++nq) {
    const float lt = l[nq] + __shfl_xor(l[nq], 32, 64);
    const float inv = 1.f / lt;
    if (!live[nq]) continue;
    uint16_t *op = out_at(nq);
#pragma unroll
    for (int md = 0; md < 4; ++md)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f32x8 v8;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v8[i] = o[md][nq][4 * j + i] * inv;
          v8[4 + i] = 0.f;
        }
        const bf16x8 w8 = __builtin_convertvector(v8, bf16x8);
        const bf16x4 w4 = __builtin_shufflevector(w8, w8, 0, 1, 2, 3);
        *reinterpret_cast<uint2 *>(op + 32 * md + 8 * j + 4 * h) = __builtin_bit_cast(uint2, w4);
      }
  }
}

}  // namespace

bool prefill_mfma_supported(const AttnArgs &a) {
  return a.dtype == MCAMD_BF16 && a.head_dim == D && a.n_head / a.n_kv_head <= kPairs;
}

int launch_prefill_mfma(const AttnArgs &a) {
  MfmaParams P;
  P.q = static_cast<const uint16_t *>(a.q);
  P.k_cache = static_cast<const uint16_t *>(a.k_cache);
  P.v_cache = static_cast<const uint16_t *>(a.v_cache);
  P.seqlens = a.seqlens;
  P.out = static_cast<uint16_t *>(a.out);
  P.T_new = int(a.t_new);
  P.H = int(a.n_head);
  P.H_kv = int(a.n_kv_head);
  P.G = int(a.n_head / a.n_kv_head);
  P.QT = kPairs / P.G;
  P.T_max = int(a.t_max);
  P.window = int(a.window < 0 ? -1 : a.window);
  P.n_bh = int(a.batch * a.n_kv_head);
  P.cache_b = a.cache_batch_stride;
  P.scale_log2 = float(kLog2e / std::sqrt(double(D)));
  const int64_t n_qt = (a.t_new + P.QT - 1) / P.QT;
  const int64_t blocks = n_qt * P.n_bh;
  if (blocks > 0x7fffffff) return fail(MCAMD_EUNSUPPORTED, "prefill: grid too large");
  hipLaunchKernelGGL(prefill_mfma_kernel, dim3(unsigned(blocks)), dim3(256), 0, a.stream, P);
  return launch_status("prefill_mfma");
}

}  // namespace mcamd
