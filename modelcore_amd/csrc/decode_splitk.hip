// Single-token decode attention over the KV cache, as split-K flash-decoding.
//
// Semantics: modelcore/kernels/flash_attn.py:348-366 with T_new == 1. The query of row b sits at
// p = cache_seqlens[b] and attends keys [lo, p], lo = max(0, p - window) (window < 0: lo = 0),
// which is both the sliced uniform path (:217-224) and the ragged mask (:246-264). Query head h
// reads KV head h / G, G = H / H_kv (SDPA enable_gqa). Scale 1/sqrt(D).
//
// Work split. The key range of a row is cut into splits of kDecodeSplitLen keys, aligned to lo.
// One workgroup owns (row b, KV head, split) and serves every query head of that KV head's GQA
// group (up to GM at a time), so each K/V byte of the split is read from HBM once. The grid is
// sized from T_max (no host sync on cache_seqlens); splits past a row's length exit at once.
//
// Inside a workgroup (256 threads): LPT = D / VEC lanes cover one key's D elements with one
// 16-byte load each, so a wave reads 64/LPT whole head rows per instruction. Pass 1 forms the
// G scores of every key of the split (lane partial dots, then a butterfly over the LPT lanes)
// into LDS; pass 2 takes the exact split maximum and the exp2 weights per head; pass 3 streams V
// and accumulates the weighted rows, which are summed over the key groups with wave shuffles
// and over the four waves through LDS. The split's (m, l, o[D]) go to the workspace; the combine
// kernel merges the splits of a (row, head) by log-sum-exp.
#include "kernels.h"

#include <cmath>

namespace mcamd {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int SL = kDecodeSplitLen;

struct DecodeParams {
  const void *q, *k_new, *v_new, *k_cache, *v_cache;
  const int32_t *seqlens;
  void *out;
  float *part_o;   // [B][H][n_splits][D]
  float *part_ml;  // [B][H][n_splits][2]
  int H, H_kv, G, n_hchunks, T_max, window, n_splits, D;
  int64_t cache_b;
  float scale_log2;
};

// DP is head_dim rounded up to a power of two (at least 16): LPT = DP / VEC lanes cover one key
// row, and lanes past the real head_dim D hold nothing (they load no data and add zeros).
template <class E, int DP, int GM>
__global__ __launch_bounds__(kThreads) void decode_split_kernel(DecodeParams P) {
  constexpr int VEC = Vec<E>::N;
  constexpr int LPT = DP / VEC;        // lanes per key row
  constexpr int TPI = kThreads / LPT;  // keys per pass of the workgroup
  constexpr int U = 4;                 // keys in flight per thread
  static_assert(LPT >= 1 && LPT <= 64 && (64 % LPT) == 0, "head_dim too large for one wave");
  const int D = P.D;

  __shared__ float s_p[GM][SL];
  __shared__ float s_m[GM], s_l[GM];
  __shared__ float s_red[kWaves][GM][DP];

  const int split = blockIdx.x;
  const int kvh = blockIdx.y / P.n_hchunks;
  const int hc = blockIdx.y - kvh * P.n_hchunks;
  const int b = blockIdx.z;
  const int h0 = kvh * P.G + hc * GM;
  const int gcount = min(GM, P.G - hc * GM);

  const int pos = P.seqlens[b];
  if (pos < 0 || pos >= P.T_max) return;  // the combine writes NaN for this row
  const int lo = key_lo(pos, P.window);
  const int t0 = lo + split * SL;
  if (t0 > pos) return;
  const int n = min(SL, pos - t0 + 1);

  const int tid = threadIdx.x;
  const int li = tid % LPT;
  const int tg = tid / LPT;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const bool live = li * VEC < D;  // this lane holds dims of the head

  const E *q = static_cast<const E *>(P.q);
  const E *kc = static_cast<const E *>(P.k_cache);
  const E *vc = static_cast<const E *>(P.v_cache);
  const E *kn = static_cast<const E *>(P.k_new);
  const E *vn = static_cast<const E *>(P.v_new);
  const int64_t row_base = int64_t(b) * P.cache_b + int64_t(kvh) * D + li * VEC;
  const int64_t tok_stride = int64_t(P.H_kv) * D;
  const int64_t new_off = (int64_t(b) * P.H_kv + kvh) * D + li * VEC;

  float qv[GM][VEC];
#pragma unroll
  for (int g = 0; g < GM; ++g) {
    if (g < gcount && live) {
      float x[VEC];
      Vec<E>::load(q + (int64_t(b) * P.H + h0 + g) * D + li * VEC, x);
#pragma unroll
      for (int e = 0; e < VEC; ++e) qv[g][e] = x[e] * P.scale_log2;
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) qv[g][e] = 0.f;
    }
  }

  // Pass 1: scores (already in log2 units) of every key of the split.
  for (int r0 = tg; r0 < n; r0 += TPI * U) {
    float kx[U][VEC];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r = r0 + u * TPI;
      if (r < n && live) {
        const int t = t0 + r;
        const E *src = (t == pos && kn) ? kn + new_off : kc + row_base + int64_t(t) * tok_stride;
        Vec<E>::unpack(load_stream(src), kx[u]);  // K/V are read once per pass
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) kx[u][e] = 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r = r0 + u * TPI;
      float acc[GM];
#pragma unroll
      for (int g = 0; g < GM; ++g) {
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < VEC; ++e) s = fmaf(qv[g][e], kx[u][e], s);
        acc[g] = wave_sum<LPT>(s);
      }
      if (li == 0 && r < n) {
#pragma unroll
        for (int g = 0; g < GM; ++g) s_p[g][r] = acc[g];
      }
    }
  }
  __syncthreads();

  // Pass 2: exact maximum of the split and exp2 weights, one wave per head.
  for (int g = wave; g < gcount; g += kWaves) {
    float m = -INFINITY;
    for (int i = lane; i < n; i += 64) m = fmaxf(m, s_p[g][i]);
    m = wave_max<64>(m);
    float l = 0.f;
    for (int i = lane; i < n; i += 64) {
      const float p = fast_exp2(s_p[g][i] - m);
      s_p[g][i] = p;
      l += p;
    }
    l = wave_sum<64>(l);
    if (lane == 0) {
      s_m[g] = m;
      s_l[g] = l;
    }
  }
  __syncthreads();

  // Pass 3: weighted sum of the split's value rows.
  float o[GM][VEC];
#pragma unroll
  for (int g = 0; g < GM; ++g)
#pragma unroll
    for (int e = 0; e < VEC; ++e) o[g][e] = 0.f;

  for (int r0 = tg; r0 < n; r0 += TPI * U) {
    float vx[U][VEC];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r = r0 + u * TPI;
      if (r < n && live) {
        const int t = t0 + r;
        const E *src = (t == pos && vn) ? vn + new_off : vc + row_base + int64_t(t) * tok_stride;
        Vec<E>::unpack(load_stream(src), vx[u]);  // K/V are read once per pass
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) vx[u][e] = 0.f;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r = r0 + u * TPI;
      if (r < n) {
#pragma unroll
        for (int g = 0; g < GM; ++g) {
          const float p = s_p[g][r];
#pragma unroll
          for (int e = 0; e < VEC; ++e) o[g][e] = fmaf(p, vx[u][e], o[g][e]);
        }
      }
    }
  }

  // Sum over the key groups of a wave (lanes li, li + LPT, ...), then over the waves.
#pragma unroll
  for (int g = 0; g < GM; ++g)
#pragma unroll
    for (int e = 0; e < VEC; ++e)
#pragma unroll
      for (int off = LPT; off < 64; off <<= 1) o[g][e] += __shfl_xor(o[g][e], off, 64);
  if (lane < LPT) {
#pragma unroll
    for (int g = 0; g < GM; ++g)
#pragma unroll
      for (int e = 0; e < VEC; ++e) s_red[wave][g][li * VEC + e] = o[g][e];
  }
  __syncthreads();

  const int64_t base = (int64_t(b) * P.H + h0) * P.n_splits + split;
  for (int i = tid; i < gcount * D; i += kThreads) {
    const int g = i / D;
    const int d = i - g * D;
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) s += s_red[w][g][d];
    P.part_o[(base + int64_t(g) * P.n_splits) * D + d] = s;
  }
  if (tid < gcount) {
    P.part_ml[(base + int64_t(tid) * P.n_splits) * 2 + 0] = s_m[tid];
    P.part_ml[(base + int64_t(tid) * P.n_splits) * 2 + 1] = s_l[tid];
  }
}

// Merge of the splits of one (row, head): out = sum_s o_s 2^(m_s - M) / sum_s l_s 2^(m_s - M).
template <class E>
__global__ __launch_bounds__(128) void decode_combine_kernel(DecodeParams P) {
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int D = P.D;
  E *out = static_cast<E *>(P.out) + (int64_t(b) * P.H + h) * D;
  const int pos = P.seqlens[b];
  if (pos < 0 || pos >= P.T_max) {
    for (int d = threadIdx.x; d < D; d += blockDim.x) out[d] = from_f32<E>(NAN);
    return;
  }
  const int lo = key_lo(pos, P.window);
  const int ns = (pos - lo + 1 + SL - 1) / SL;
  const int64_t base = (int64_t(b) * P.H + h) * P.n_splits;
  const float *ml = P.part_ml + base * 2;
  float M = -INFINITY;
  for (int s = 0; s < ns; ++s) M = fmaxf(M, ml[2 * s]);
  float L = 0.f;
  for (int s = 0; s < ns; ++s) L += ml[2 * s + 1] * fast_exp2(ml[2 * s] - M);
  const float inv = 1.f / L;
  const float *po = P.part_o + base * D;
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float acc = 0.f;
    for (int s = 0; s < ns; ++s) acc = fmaf(po[int64_t(s) * D + d], fast_exp2(ml[2 * s] - M), acc);
    out[d] = from_f32<E>(acc * inv);
  }
}

template <class E, int DP, int GM>
int run_decode(const DecodeParams &P, int B, hipStream_t stream) {
  dim3 grid(P.n_splits, P.H_kv * P.n_hchunks, B);
  hipLaunchKernelGGL((decode_split_kernel<E, DP, GM>), grid, dim3(kThreads), 0, stream, P);
  int st = launch_status("decode_split");
  if (st != MCAMD_OK) return st;
  hipLaunchKernelGGL(decode_combine_kernel<E>, dim3(P.H, B), dim3(128), 0, stream, P);
  return launch_status("decode_combine");
}

template <class E, int DP>
int dispatch_gm(DecodeParams &P, int B, hipStream_t s) {
  if (P.G == 1) { P.n_hchunks = 1; return run_decode<E, DP, 1>(P, B, s); }
  if (P.G == 2) { P.n_hchunks = 1; return run_decode<E, DP, 2>(P, B, s); }
  if (P.G <= 4) { P.n_hchunks = 1; return run_decode<E, DP, 4>(P, B, s); }
  P.n_hchunks = (P.G + 7) / 8;
  return run_decode<E, DP, 8>(P, B, s);
}

// Any head_dim up to 256 whose rows are whole 16-byte vectors (checked before; wider heads take
// the general prefill kernel, see launch_decode), run in the
// instantiation of the next power of two.
template <class E>
int dispatch_d(DecodeParams &P, int B, hipStream_t s) {
  switch (head_dim_bucket(P.D)) {
    case 16: return dispatch_gm<E, 16>(P, B, s);
    case 32: return dispatch_gm<E, 32>(P, B, s);
    case 64: return dispatch_gm<E, 64>(P, B, s);
    case 128: return dispatch_gm<E, 128>(P, B, s);
    case 256: return dispatch_gm<E, 256>(P, B, s);
    default:
      return fail(MCAMD_EUNSUPPORTED, "decode: head_dim must be at most 256");
  }
}

}  // namespace

int64_t decode_max_splits(int64_t t_max, int64_t window) {
  const int64_t span = window >= 0 ? std::min<int64_t>(t_max, window + 1) : t_max;
  return (span + SL - 1) / SL;
}

size_t decode_workspace_bytes(int64_t batch, int64_t n_head, int64_t n_kv_head, int64_t head_dim,
                              int64_t t_max, int64_t window) {
  const int64_t ns = decode_max_splits(t_max, window);
  // Head dims above 256 take the general prefill kernel, which needs no workspace.
  const size_t generic = head_dim > 256 ? 0 : size_t(batch * n_head * ns * (head_dim + 2) * 4);
  // The fused path serves head_dim 128 (bf16); other head dims only ever take the general one.
  const size_t fused =
      head_dim == 128 ? decode_fused_partial_bytes(batch, n_head, n_kv_head, t_max, window) : 0;
  const size_t part = generic > fused ? generic : fused;
  return (part + 255) / 256 * 256;
}

int launch_decode(const AttnArgs &a) {
  int st = check_attn_shapes(a, true);
  if (st != MCAMD_OK) return st;
  if (a.t_new != 1) return fail(MCAMD_EINVAL, "decode: t_new must be 1");
  if (a.batch == 0) {
    clear_error();
    return MCAMD_OK;
  }
  if (decode_fused_supported(a)) return launch_decode_fused(a);
  if (a.k_new) {
    // The general-shape kernels read the cache only: append first.
    AppendArgs ap{a.k_new, a.v_new, const_cast<void *>(a.k_cache), const_cast<void *>(a.v_cache),
                  a.seqlens, a.batch, 1, a.n_kv_head, a.head_dim, a.t_max, a.cache_batch_stride,
                  a.dtype, a.stream};
    st = launch_append(ap);
    if (st != MCAMD_OK) return st;
  }
  if (a.head_dim > 256) {
    // Past 256 an fp32 key row needs more than a wave's 64 lanes of 16 bytes, and the cross-wave
    // sum buffer (4 x GM x D floats) outgrows the LDS budget: the general prefill kernel (one
    // query per row here) walks the keys instead, with no split and no workspace.
    AttnArgs pa = a;
    pa.k_new = pa.v_new = nullptr;  // appended above
    st = launch_prefill_generic(pa);
    if (st != MCAMD_OK || !a.advance_seqlens) return st;
    return launch_advance(a.advance_seqlens, a.batch, a.advance, a.stream);
  }
  DecodeParams P;
  P.q = a.q;
  P.k_new = a.k_new;
  P.v_new = a.v_new;
  P.k_cache = a.k_cache;
  P.v_cache = a.v_cache;
  P.seqlens = a.seqlens;
  P.out = a.out;
  P.H = int(a.n_head);
  P.H_kv = int(a.n_kv_head);
  P.G = int(a.n_head / a.n_kv_head);
  P.n_hchunks = 1;
  P.T_max = int(a.t_max);
  P.window = int(a.window < 0 ? -1 : a.window);
  P.n_splits = int(decode_max_splits(a.t_max, a.window));
  P.D = int(a.head_dim);
  P.cache_b = a.cache_batch_stride;
  P.scale_log2 = float(kLog2e / std::sqrt(double(a.head_dim)));
  const int64_t floats_o = a.batch * a.n_head * P.n_splits * a.head_dim;
  P.k_new = P.v_new = nullptr;  // appended above
  P.part_o = static_cast<float *>(a.workspace);
  P.part_ml = P.part_o + floats_o;
  st = a.dtype == MCAMD_BF16 ? dispatch_d<bf16>(P, int(a.batch), a.stream)
                             : dispatch_d<float>(P, int(a.batch), a.stream);
  if (st != MCAMD_OK || !a.advance_seqlens) return st;
  return launch_advance(a.advance_seqlens, a.batch, a.advance, a.stream);
}

}  // namespace mcamd
