// Multi-token attention against the cache prefix, any head_dim up to 256 made of whole 16-byte
// vectors, bf16 or fp32.
//
// Semantics: modelcore/kernels/flash_attn.py:226-244 (uniform, explicit mask with row offset
// Tk - Tq) and :362-364 (ragged mask). Query t of row b sits at p = cache_seqlens[b] + t and
// attends keys col <= p with p - col <= window when window >= 0. The cache already holds the new
// tokens (the append runs first), so the prefix includes the chunk itself.
//
// This is the general-shape kernel (fp32 caches, small or odd head counts and head dims); the bf16
// MFMA kernel in prefill_mfma.hip takes the large shapes. One workgroup owns 64 (query, head)
// rows of one KV head: 64 / G consecutive queries times the G query heads that share the KV head,
// so every K/V tile staged in LDS serves all of them. Four lanes share a row, each owning every
// fourth dimension (of the head_dim rounded up to a power of two; dims past the real head_dim
// stay zero). Keys are walked in tiles of 32 from the first key any row of the block can see to
// the last; each tile's scores are masked per row, and an online softmax (running max m,
// running sum l, rescaled accumulator) folds the tile in.
#include "kernels.h"

#include <cmath>

namespace mcamd {
namespace {

constexpr int kThreads = 256;
constexpr int kRows = 64;
// Keys per LDS tile: 32, or 16 for head dims above 256 (K and V tiles of 64 KiB in fp32).
template <int DP>
constexpr int kTileKeys = DP <= 256 ? 32 : 16;

struct PrefillParams {
  const void *q, *k_cache, *v_cache;
  const int32_t *seqlens;
  const int32_t *rows, *cu;  // varlen (optional): cache row and token range per sequence
  void *out;
  int T_new, H, H_kv, G, QT, T_max, window, D;
  int64_t cache_b;
  float scale_log2;
};

template <class E, int DP>
__global__ __launch_bounds__(kThreads) void prefill_generic_kernel(PrefillParams P) {
  constexpr int DS = DP / 4;  // dimensions per lane (lane j owns d = 4*i + j, d < DP)
  constexpr int KT = kTileKeys<DP>;
  constexpr int VEC = Vec<E>::N;
  const int D = P.D;          // the real head_dim (<= DP); dims past it are zero in LDS and q
  __shared__ float sk[KT][DP];
  __shared__ float sv[KT][DP];

  const int qt0 = blockIdx.x * P.QT;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;  // sequence; varlen: tokens [cu[b], cu[b + 1]) in cache row rows[b]
  const int crow = P.rows ? P.rows[b] : b;
  const int64_t tok0 = P.cu ? int64_t(P.cu[b]) : int64_t(b) * P.T_new;
  const int T_b = P.cu ? P.cu[b + 1] - P.cu[b] : P.T_new;
  if (qt0 >= T_b) return;  // a query tile past a shorter sequence's end (whole workgroup)
  const int tid = threadIdx.x;
  const int row = tid >> 2;
  const int j = tid & 3;
  const int tq = qt0 + row / P.G;
  const int g = row - (row / P.G) * P.G;
  const int h = kvh * P.G + g;
  const bool active = (row < P.QT * P.G) && (tq < T_b);

  const int pos = P.seqlens[crow];
  const int q_last = min(qt0 + P.QT, T_b) - 1;
  const bool row_ok = pos >= 0 && pos + T_b <= P.T_max;

  const E *q = static_cast<const E *>(P.q);
  E *out = static_cast<E *>(P.out);
  const int64_t out_off = ((tok0 + tq) * P.H + h) * D;

  if (!row_ok) {
    if (active)
      for (int i = 0; i < DS; ++i)
        if (4 * i + j < D) out[out_off + 4 * i + j] = from_f32<E>(NAN);
    return;
  }
  // Columns past the head_dim: zero once; the tile staging below writes columns < D only.
  if (D < DP)
    for (int c = tid; c < KT * DP; c += kThreads)
      if (c % DP >= D) {
        sk[c / DP][c % DP] = 0.f;
        sv[c / DP][c % DP] = 0.f;
      }

  const int p = pos + tq;  // this row's query position
  float qv[DS], o[DS];
#pragma unroll
  for (int i = 0; i < DS; ++i) {
    qv[i] = active && 4 * i + j < D ? to_f32<E>(q[out_off + 4 * i + j]) * P.scale_log2 : 0.f;
    o[i] = 0.f;
  }
  float m = -INFINITY, l = 0.f;

  const int p_first = pos + qt0;
  const int p_last = pos + q_last;
  const int klo = P.window >= 0 ? max(0, p_first - P.window) : 0;
  const int khi = p_last;

  const E *kc = static_cast<const E *>(P.k_cache) + int64_t(crow) * P.cache_b + int64_t(kvh) * D;
  const E *vc = static_cast<const E *>(P.v_cache) + int64_t(crow) * P.cache_b + int64_t(kvh) * D;
  const int64_t tok_stride = int64_t(P.H_kv) * D;

  for (int kt0 = klo; kt0 <= khi; kt0 += KT) {
    // Stage the K and V tile (fp32) in LDS.
    for (int c = tid; c < KT * (D / VEC); c += kThreads) {
      const int key = c / (D / VEC);
      const int dv = (c - key * (D / VEC)) * VEC;
      const int t = kt0 + key;
      float x[VEC], y[VEC];
      if (t <= khi) {
        Vec<E>::load(kc + int64_t(t) * tok_stride + dv, x);
        Vec<E>::load(vc + int64_t(t) * tok_stride + dv, y);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) x[e] = y[e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        sk[key][dv + e] = x[e];
        sv[key][dv + e] = y[e];
      }
    }
    __syncthreads();

    float sc[KT];
    float mt = -INFINITY;
#pragma unroll
    for (int kk = 0; kk < KT; ++kk) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < DS; ++i) s = fmaf(qv[i], sk[kk][4 * i + j], s);
      s += __shfl_xor(s, 1, 64);
      s += __shfl_xor(s, 2, 64);
      const int col = kt0 + kk;
      const bool ok = active && col <= p && (P.window < 0 || p - col <= P.window);
      sc[kk] = ok ? s : -INFINITY;
      mt = fmaxf(mt, sc[kk]);
    }
    if (mt > -INFINITY) {
      const float m_new = fmaxf(m, mt);
      const float corr = fast_exp2(m - m_new);
      l *= corr;
#pragma unroll
      for (int i = 0; i < DS; ++i) o[i] *= corr;
#pragma unroll
      for (int kk = 0; kk < KT; ++kk) {
        if (sc[kk] > -INFINITY) {
          const float pk = fast_exp2(sc[kk] - m_new);
          l += pk;
#pragma unroll
          for (int i = 0; i < DS; ++i) o[i] = fmaf(pk, sv[kk][4 * i + j], o[i]);
        }
      }
      m = m_new;
    }
    __syncthreads();
  }

  if (active) {
    const float inv = 1.f / l;
#pragma unroll
    for (int i = 0; i < DS; ++i)
      if (4 * i + j < D) out[out_off + 4 * i + j] = from_f32<E>(o[i] * inv);
  }
}

template <class E, int DP>
int run_prefill(const PrefillParams &P, int B, hipStream_t stream) {
  dim3 grid((P.T_new + P.QT - 1) / P.QT, P.H_kv, B);
  hipLaunchKernelGGL((prefill_generic_kernel<E, DP>), grid, dim3(kThreads), 0, stream, P);
  return launch_status("prefill_generic");
}

template <class E>
int dispatch_d(const PrefillParams &P, int D, int B, hipStream_t s) {
  switch (head_dim_bucket(D)) {
    case 16: return run_prefill<E, 16>(P, B, s);
    case 32: return run_prefill<E, 32>(P, B, s);
    case 64: return run_prefill<E, 64>(P, B, s);
    case 128: return run_prefill<E, 128>(P, B, s);
    case 256: return run_prefill<E, 256>(P, B, s);
    case 512: return run_prefill<E, 512>(P, B, s);
    default:
      return fail(MCAMD_EUNSUPPORTED, "attention: head_dim must be at most 512");
  }
}

}  // namespace

int launch_prefill_generic(const AttnArgs &a) {
  PrefillParams P;
  P.q = a.q;
  P.k_cache = a.k_cache;
  P.v_cache = a.v_cache;
  P.seqlens = a.seqlens;
  P.rows = a.rows;
  P.cu = a.cu;
  P.out = a.out;
  P.T_new = int(a.t_new);
  P.H = int(a.n_head);
  P.H_kv = int(a.n_kv_head);
  P.G = int(a.n_head / a.n_kv_head);
  if (P.G > kRows) return fail(MCAMD_EUNSUPPORTED, "prefill: more than 64 query heads per KV head");
  P.QT = kRows / P.G;
  P.T_max = int(a.t_max);
  P.window = int(a.window < 0 ? -1 : a.window);
  P.cache_b = a.cache_batch_stride;
  P.D = int(a.head_dim);
  P.scale_log2 = float(kLog2e / std::sqrt(double(a.head_dim)));
  if (a.dtype == MCAMD_BF16) return dispatch_d<bf16>(P, int(a.head_dim), int(a.batch), a.stream);
  return dispatch_d<float>(P, int(a.head_dim), int(a.batch), a.stream);
}

int launch_prefill(const AttnArgs &a) {
  int st = check_attn_shapes(a, false);
  if (st != MCAMD_OK) return st;
  if (a.t_new < 1) return fail(MCAMD_EINVAL, "prefill: t_new must be >= 1");
  if (a.batch == 0) {
    clear_error();
    return MCAMD_OK;
  }
  if (prefill_mfma_supported(a)) return launch_prefill_mfma(a);
  return launch_prefill_generic(a);
}

}  // namespace mcamd
