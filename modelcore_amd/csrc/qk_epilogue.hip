// The step before the cached attention, fused: RoPE, QK RMS-norm and the x1.2 scale of q and k,
// then the append of k and v into the cache -- one launch instead of about ten elementwise
// kernels and the append.
//
// Semantics, per token t of row b at position p = cache_seqlens[b] + t (the row's position
// before this call plus t; modelcore/components/rotary.py:50-67), for every query head of q and
// every KV head of k (modelcore/components/attention.py:143-150):
//   rope  (modelcore/components/rope.py:4-12): with c = cos[p, j], s = sin[p, j], j < D/2,
//           y[j]       = x[j] * c + x[j + D/2] * s
//           y[j + D/2] = x[j] * (-s) + x[j + D/2] * c
//         each product and sum rounded to the storage dtype, as the elementwise torch ops do;
//   norm  (modelcore/components/norm.py:43-44, F.rms_norm without weight): in fp32,
//           z = y * (1 / sqrt(mean(y^2) + eps)), rounded to the storage dtype;
//   scale: out = z * scale (1.2 in the model) in fp32, rounded to the storage dtype.
// q, k and v may be strided views (a fused QKV projection's output): tokens are `*_token_stride`
// elements apart, heads contiguous within a token. q's result goes to q_out (contiguous); k's
// result and v (unchanged) go to k_cache / v_cache at p
// (modelcore/kernels/flash_attn.py:336-346). With k = v = null only q is transformed: the
// KV-sharing consumer layers (attention.py:152-157).
//
// The only difference from the unfused torch ops is the order of the fp32 sum of squares, which
// can move a result by one unit in the last place of the storage dtype.
//
// One wave per (token, head item); lane i holds dims j and j + D/2 for j = i (and i + 64 when
// D > 128), so the rotation pairs sit in one lane and the sum of squares is one wave reduction.
// Positions outside the rotary table or the cache leave the cache untouched and write NaN to
// q_out (the callers check positions on the host first, as the reference does).
#include "kernels.h"

#include <cmath>

namespace mcamd {
namespace {

constexpr int kWavesPerBlock = 4;

// Round-to-nearest-even to bf16, returned as float; NaN becomes the canonical quiet NaN.
__device__ __forceinline__ float round_bf16(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return __uint_as_float(0x7fc00000u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return __uint_as_float(u & 0xffff0000u);
}

template <bool BF16>
struct Elem;
template <>
struct Elem<true> {
  typedef uint16_t T;
  static __device__ __forceinline__ float load(const T *p) {
    return __uint_as_float(uint32_t(*p) << 16);
  }
  static __device__ __forceinline__ void store(T *p, float x) {
    *p = uint16_t(__float_as_uint(round_bf16(x)) >> 16);
  }
  static __device__ __forceinline__ float rnd(float x) { return round_bf16(x); }
};
template <>
struct Elem<false> {
  typedef float T;
  static __device__ __forceinline__ float load(const T *p) { return *p; }
  static __device__ __forceinline__ void store(T *p, float x) { *p = x; }
  static __device__ __forceinline__ float rnd(float x) { return x; }
};

struct EpiParams {
  const void *q, *k, *v, *cos, *sin;
  void *k_cache, *v_cache, *q_out;
  const int32_t *seqlens;
  int64_t n_tokens, n_pos, t_max, cache_b;
  int64_t q_tok, k_tok, v_tok;  // elements between consecutive tokens of q, k, v
  int t_new, H, H_kv, D, n_items;
  float eps, scale;
  // Or, instead of q, k, v: the unsummed K-split partials of the stacked QKV projection,
  // (part_S, n_tokens, part_tok) fp32, q / k / v at columns 0, H D, (H + H_kv) D of a row; each
  // value is their in-order sum rounded to bf16, as the GEMM's own reduce pass makes it.
  const float *part;
  int64_t part_tok, part_slice;
  int part_S;
};

// The leading arguments repeat the fields of P that the first loads need (the row's position,
// then its source row), so that they arrive preloaded in SGPRs at dispatch (the library is
// built with kernarg preloading, which covers scalar arguments only).
template <bool BF16>
__global__ __launch_bounds__(64 * kWavesPerBlock) void qk_epilogue_kernel(
    const int32_t *a_seqlens, const float *a_part, int64_t a_part_tok, int64_t a_n_tokens,
    int a_n_items, int a_t_new, int a_D, int a_H, int a_H_kv, EpiParams P) {
  // Every product and sum is rounded on its own, as the separate torch kernels do.
#pragma clang fp contract(off)
  P.seqlens = a_seqlens;
  P.part = a_part;
  P.part_tok = a_part_tok;
  P.n_tokens = a_n_tokens;
  P.n_items = a_n_items;
  P.t_new = a_t_new;
  P.D = a_D;
  P.H = a_H;
  P.H_kv = a_H_kv;
  typedef Elem<BF16> E;
  typedef typename E::T T;
  const int lane = threadIdx.x & 63;
  const int64_t w = int64_t(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
  const int64_t tok = w / P.n_items;
  if (tok >= P.n_tokens) return;
  const int item = int(w - tok * P.n_items);
  const int b = int(tok / P.t_new);
  const int t = int(tok - int64_t(b) * P.t_new);
  const int64_t pos = int64_t(P.seqlens[b]) + t;
  const int half = P.D >> 1;
  const bool in_table = pos >= 0 && pos < P.n_pos;
  const bool in_cache = pos >= 0 && pos < P.t_max;

  // Element j of this item's source row, from q/k/v or from the projection's partials (whose
  // columns follow the item order: H query heads, then H_kv key heads, then H_kv value heads).
  const float *psrc = P.part ? P.part + tok * P.part_tok + int64_t(item) * P.D : nullptr;
  auto part_load = [&](int j) {
    float a = 0.f;
    for (int s = 0; s < P.part_S; ++s) a += psrc[int64_t(s) * P.part_slice + j];
    return round_bf16(a);
  };

  if (item >= P.H + P.H_kv) {  // v: plain copy into the cache
    if (!in_cache) return;
    const int hk = item - P.H - P.H_kv;
    T *dst = static_cast<T *>(P.v_cache) + int64_t(b) * P.cache_b + (pos * P.H_kv + hk) * P.D;
    if (psrc) {
      for (int d = lane; d < P.D; d += 64) E::store(dst + d, part_load(d));
      return;
    }
    const T *src = static_cast<const T *>(P.v) + tok * P.v_tok + int64_t(hk) * P.D;
    for (int d = lane; d < P.D; d += 64) dst[d] = src[d];
    return;
  }
  const bool is_q = item < P.H;
  const T *src = psrc ? nullptr
                 : is_q ? static_cast<const T *>(P.q) + tok * P.q_tok + int64_t(item) * P.D
                        : static_cast<const T *>(P.k) + tok * P.k_tok + int64_t(item - P.H) * P.D;
  auto load = [&](int j) { return psrc ? part_load(j) : E::load(src + j); };
  T *dst;
  if (is_q) {
    dst = static_cast<T *>(P.q_out) + (tok * P.H + item) * P.D;
    if (!in_table) {
      for (int d = lane; d < P.D; d += 64) E::store(dst + d, NAN);
      return;
    }
  } else {
    if (!in_table || !in_cache) return;
    dst = static_cast<T *>(P.k_cache) + int64_t(b) * P.cache_b +
          (pos * P.H_kv + (item - P.H)) * P.D;
  }
  const T *cs = static_cast<const T *>(P.cos) + pos * half;
  const T *sn = static_cast<const T *>(P.sin) + pos * half;

  float y1[2] = {0.f, 0.f}, y2[2] = {0.f, 0.f};
  float ss = 0.f;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int j = lane + 64 * r;
    if (j < half) {
      const float x1 = load(j), x2 = load(j + half);
      const float c = E::load(cs + j), s = E::load(sn + j);
      y1[r] = E::rnd(E::rnd(x1 * c) + E::rnd(x2 * s));
      y2[r] = E::rnd(E::rnd(x1 * -s) + E::rnd(x2 * c));
      ss = fmaf(y1[r], y1[r], ss);
      ss = fmaf(y2[r], y2[r], ss);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
  const float inv = __fdiv_rn(1.f, __fsqrt_rn(__fdiv_rn(ss, float(P.D)) + P.eps));
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int j = lane + 64 * r;
    if (j < half) {
      E::store(dst + j, E::rnd(y1[r] * inv) * P.scale);
      E::store(dst + j + half, E::rnd(y2[r] * inv) * P.scale);
    }
  }
}

}  // namespace
}  // namespace mcamd

using namespace mcamd;

extern "C" int mcamd_qk_rope_norm_append(const void *q, int64_t q_token_stride, const void *k,
                                         int64_t k_token_stride, const void *v,
                                         int64_t v_token_stride, const void *cos,
                                         const void *sin, int64_t n_pos,
                                         void *k_cache, void *v_cache,
                                         const int32_t *cache_seqlens, void *q_out,
                                         int64_t batch, int64_t t_new, int64_t n_head,
                                         int64_t n_kv_head, int64_t head_dim, int64_t t_max,
                                         int64_t cache_batch_stride, float eps, float scale,
                                         int dtype, void *stream) {
  if (dtype != MCAMD_F32 && dtype != MCAMD_BF16)
    return fail(MCAMD_EINVAL, "qk_rope_norm_append: dtype must be MCAMD_F32 or MCAMD_BF16");
  if (batch < 0 || t_new < 0 || n_head <= 0 || n_kv_head <= 0 || n_pos <= 0)
    return fail(MCAMD_EINVAL, "qk_rope_norm_append: sizes must be positive (batch, t_new may be 0)");
  if (head_dim <= 0 || head_dim % 2 != 0 || head_dim > 256)
    return fail(MCAMD_EUNSUPPORTED, "qk_rope_norm_append: head_dim must be even and <= 256");
  if ((k == nullptr) != (v == nullptr))
    return fail(MCAMD_EINVAL, "qk_rope_norm_append: pass both k and v, or neither");
  if (!(eps >= 0.f) || !std::isfinite(scale))
    return fail(MCAMD_EINVAL, "qk_rope_norm_append: eps must be >= 0 and scale finite");
  const bool with_kv = k != nullptr;
  if (batch * t_new == 0) {
    clear_error();
    return MCAMD_OK;
  }
  if (!q || !cos || !sin || !cache_seqlens || !q_out ||
      (with_kv && (!k_cache || !v_cache || t_max <= 0)))
    return fail(MCAMD_EINVAL, "qk_rope_norm_append: null pointer or empty cache");
  if (with_kv && cache_batch_stride < t_max * n_kv_head * head_dim)
    return fail(MCAMD_EINVAL, "qk_rope_norm_append: cache_batch_stride smaller than T_max*H_kv*D");
  if (q_token_stride < n_head * head_dim ||
      (with_kv && (k_token_stride < n_kv_head * head_dim || v_token_stride < n_kv_head * head_dim)))
    return fail(MCAMD_EINVAL, "qk_rope_norm_append: a token stride is smaller than heads * head_dim");
  EpiParams P{};
  P.q = q;
  P.k = k;
  P.v = v;
  P.cos = cos;
  P.sin = sin;
  P.k_cache = k_cache;
  P.v_cache = v_cache;
  P.q_out = q_out;
  P.q_tok = q_token_stride;
  P.k_tok = k_token_stride;
  P.v_tok = v_token_stride;
  P.seqlens = cache_seqlens;
  P.n_tokens = batch * t_new;
  P.n_pos = n_pos;
  P.t_max = with_kv ? t_max : 0;
  P.cache_b = cache_batch_stride;
  P.t_new = int(t_new);
  P.H = int(n_head);
  P.H_kv = int(n_kv_head);
  P.D = int(head_dim);
  P.n_items = int(n_head + (with_kv ? 2 * n_kv_head : 0));
  P.eps = eps;
  P.scale = scale;
  if (t_new > 0x7fffffff || n_head + 2 * n_kv_head > 0x7fffffff)
    return fail(MCAMD_EUNSUPPORTED, "qk_rope_norm_append: sizes too large");
  const int64_t waves = P.n_tokens * P.n_items;
  const int64_t blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
  if (blocks > 0x7fffffff) return fail(MCAMD_EUNSUPPORTED, "qk_rope_norm_append: grid too large");
  if (dtype == MCAMD_BF16)
    hipLaunchKernelGGL(qk_epilogue_kernel<true>, dim3(unsigned(blocks)), dim3(64 * kWavesPerBlock),
                       0, as_stream(stream), P.seqlens, P.part, P.part_tok, P.n_tokens,
                       P.n_items, P.t_new, P.D, P.H, P.H_kv, P);
  else
    hipLaunchKernelGGL(qk_epilogue_kernel<false>, dim3(unsigned(blocks)),
                       dim3(64 * kWavesPerBlock), 0, as_stream(stream), P.seqlens, P.part, P.part_tok, P.n_tokens,
                       P.n_items, P.t_new, P.D, P.H, P.H_kv, P);
  return launch_status("qk_rope_norm_append");
}

extern "C" int mcamd_qk_rope_norm_append_partials(
    const float *part, int64_t splits, int64_t part_token_stride, const void *cos,
    const void *sin, int64_t n_pos, void *k_cache, void *v_cache, const int32_t *cache_seqlens,
    void *q_out, int64_t batch, int64_t t_new, int64_t n_head, int64_t n_kv_head,
    int64_t head_dim, int64_t t_max, int64_t cache_batch_stride, float eps, float scale,
    int with_kv, void *stream) {
  if (batch < 0 || t_new < 0 || n_head <= 0 || n_kv_head <= 0 || n_pos <= 0)
    return fail(MCAMD_EINVAL, "qk_rope_norm_append_partials: sizes must be positive");
  if (head_dim <= 0 || head_dim % 2 != 0 || head_dim > 256)
    return fail(MCAMD_EUNSUPPORTED, "qk_rope_norm_append_partials: head_dim must be even, <= 256");
  if (splits < 1 || splits > 64)
    return fail(MCAMD_EINVAL, "qk_rope_norm_append_partials: splits must be in [1, 64]");
  if (!(eps >= 0.f) || !std::isfinite(scale))
    return fail(MCAMD_EINVAL, "qk_rope_norm_append_partials: eps must be >= 0 and scale finite");
  const int64_t width = (n_head + (with_kv ? 2 * n_kv_head : 0)) * head_dim;
  if (part_token_stride < width)
    return fail(MCAMD_EINVAL, "qk_rope_norm_append_partials: token stride smaller than the row");
  if (batch * t_new == 0) {
    clear_error();
    return MCAMD_OK;
  }
  if (!part || !cos || !sin || !cache_seqlens || !q_out ||
      (with_kv && (!k_cache || !v_cache || t_max <= 0)))
    return fail(MCAMD_EINVAL, "qk_rope_norm_append_partials: null pointer or empty cache");
  if (with_kv && cache_batch_stride < t_max * n_kv_head * head_dim)
    return fail(MCAMD_EINVAL,
                "qk_rope_norm_append_partials: cache_batch_stride smaller than T_max*H_kv*D");
  if (t_new > 0x7fffffff || n_head + 2 * n_kv_head > 0x7fffffff)
    return fail(MCAMD_EUNSUPPORTED, "qk_rope_norm_append_partials: sizes too large");
  EpiParams P{};
  P.part = part;
  P.part_S = int(splits);
  P.part_tok = part_token_stride;
  P.part_slice = batch * t_new * part_token_stride;
  P.cos = cos;
  P.sin = sin;
  P.k_cache = k_cache;
  P.v_cache = v_cache;
  P.q_out = q_out;
  P.seqlens = cache_seqlens;
  P.n_tokens = batch * t_new;
  P.n_pos = n_pos;
  P.t_max = with_kv ? t_max : 0;
  P.cache_b = cache_batch_stride;
  P.t_new = int(t_new);
  P.H = int(n_head);
  P.H_kv = int(n_kv_head);
  P.D = int(head_dim);
  P.n_items = int(n_head + (with_kv ? 2 * n_kv_head : 0));
  P.eps = eps;
  P.scale = scale;
  const int64_t waves = P.n_tokens * P.n_items;
  const int64_t blocks = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
  if (blocks > 0x7fffffff)
    return fail(MCAMD_EUNSUPPORTED, "qk_rope_norm_append_partials: grid too large");
  hipLaunchKernelGGL(qk_epilogue_kernel<true>, dim3(unsigned(blocks)), dim3(64 * kWavesPerBlock),
                     0, as_stream(stream), P.seqlens, P.part, P.part_tok, P.n_tokens,
                       P.n_items, P.t_new, P.D, P.H, P.H_kv, P);
  return launch_status("qk_rope_norm_append_partials");
}
