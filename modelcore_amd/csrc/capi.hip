// The C ABI declared in include/modelcore_amd.h: argument checks, error reporting and the
// orchestration of the cached-attention operator (append, then decode or chunked prefill).
#include "kernels.h"

#include <string>

namespace mcamd {

static thread_local std::string g_last_error;

void set_error(const std::string &msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

int check_attn_shapes(const AttnArgs &a, bool need_workspace) {
  if (a.dtype != MCAMD_F32 && a.dtype != MCAMD_BF16)
    return fail(MCAMD_EINVAL, "attention: dtype must be MCAMD_F32 or MCAMD_BF16");
  if (a.batch < 0 || a.t_new < 0 || a.n_head <= 0 || a.n_kv_head <= 0 || a.head_dim <= 0 ||
      a.t_max <= 0)
    return fail(MCAMD_EINVAL, "attention: sizes must be positive");
  if (a.n_kv_head > a.n_head || a.n_head % a.n_kv_head != 0)
    return fail(MCAMD_EINVAL, "attention: n_head must be a multiple of n_kv_head");
  if (a.t_max > (int64_t(1) << 30) || a.batch > 65535 || a.n_head > 65535)
    return fail(MCAMD_EUNSUPPORTED, "attention: sizes beyond the 32-bit index range of the kernels");
  if (a.cache_batch_stride < a.t_max * a.n_kv_head * a.head_dim)
    return fail(MCAMD_EINVAL, "attention: cache_batch_stride smaller than T_max*H_kv*D");
  if (a.batch > 0 && (!a.q || !a.k_cache || !a.v_cache || !a.seqlens || !a.out))
    return fail(MCAMD_EINVAL, "attention: null pointer");
  const size_t elem = a.dtype == MCAMD_F32 ? 4 : 2;
  if (!aligned(a.q, 16) || !aligned(a.k_cache, 16) || !aligned(a.v_cache, 16) ||
      !aligned(a.out, 16) || (a.k_new && !aligned(a.k_new, 16)) ||
      (a.v_new && !aligned(a.v_new, 16)) || (a.cache_batch_stride * elem) % 16 != 0)
    return fail(MCAMD_EINVAL, "attention: tensors must be 16-byte aligned");
  if ((a.head_dim * int64_t(elem)) % 16 != 0)
    return fail(MCAMD_EUNSUPPORTED, "attention: head_dim * itemsize must be a multiple of 16");
  if (head_dim_bucket(a.head_dim) == 0)
    return fail(MCAMD_EUNSUPPORTED, "attention: head_dim must be at most 512");
  if (need_workspace) {
    const size_t need =
        decode_workspace_bytes(a.batch, a.n_head, a.n_kv_head, a.head_dim, a.t_max, a.window);
    if (need > 0 && (!a.workspace || a.workspace_bytes < need))
      return fail(MCAMD_EWORKSPACE, "attention: workspace smaller than mcamd_attn_workspace_bytes() (" +
                                        std::to_string(need) + " bytes)");
    if (!aligned(a.workspace, 16)) return fail(MCAMD_EINVAL, "attention: workspace not 16-byte aligned");
  }
  return MCAMD_OK;
}

}  // namespace mcamd

using namespace mcamd;

extern "C" int mcamd_abi_version(void) { return 8; }

extern "C" const char *mcamd_last_error(void) { return g_last_error.c_str(); }

extern "C" int mcamd_kv_append(const void *k, const void *v, void *k_cache, void *v_cache,
                               const int32_t *cache_seqlens, int64_t batch, int64_t t_new,
                               int64_t n_kv_head, int64_t head_dim, int64_t t_max,
                               int64_t cache_batch_stride, int dtype, void *stream) {
  AppendArgs a{k,       v,      k_cache, v_cache, cache_seqlens,      batch, t_new,
               n_kv_head, head_dim, t_max, cache_batch_stride, dtype, as_stream(stream)};
  return launch_append(a);
}

extern "C" size_t mcamd_attn_workspace_bytes(int64_t batch, int64_t t_new, int64_t n_head,
                                             int64_t n_kv_head, int64_t head_dim, int64_t t_max,
                                             int64_t window) {
  if (t_new != 1 || batch <= 0 || n_kv_head <= 0 || n_head < n_kv_head) return 0;
  // Room for the shared-prefix partials too, where the fused decode can take a shared prefix on
  // the matrix cores; a workspace of decode_workspace_bytes() alone still serves every call.
  return decode_workspace_bytes(batch, n_head, n_kv_head, head_dim, t_max, window) +
         decode_prefix_bytes(batch, n_head, n_kv_head, head_dim, t_max, window);
}

extern "C" int mcamd_decode_attention(const void *q, const void *k_cache, const void *v_cache,
                                      const int32_t *cache_seqlens, void *out, int64_t batch,
                                      int64_t n_head, int64_t n_kv_head, int64_t head_dim,
                                      int64_t t_max, int64_t cache_batch_stride, int64_t window,
                                      int dtype, void *workspace, size_t workspace_bytes,
                                      void *stream) {
  AttnArgs a{q,     nullptr, nullptr, k_cache, v_cache, cache_seqlens, out,
             batch, 1,       n_head,  n_kv_head, head_dim, t_max,    cache_batch_stride,
             window, dtype,  workspace, workspace_bytes, as_stream(stream)};
  return launch_decode(a);
}

extern "C" int mcamd_prefill_attention(const void *q, const void *k_cache, const void *v_cache,
                                       const int32_t *cache_seqlens, void *out, int64_t batch,
                                       int64_t t_new, int64_t n_head, int64_t n_kv_head,
                                       int64_t head_dim, int64_t t_max,
                                       int64_t cache_batch_stride, int64_t window, int dtype,
                                       void *stream) {
  AttnArgs a{q,     nullptr, nullptr, k_cache, v_cache, cache_seqlens, out,
             batch, t_new,   n_head,  n_kv_head, head_dim, t_max,    cache_batch_stride,
             window, dtype,  nullptr, 0,        as_stream(stream)};
  return launch_prefill(a);
}

namespace {

// The cached-attention operator: append, then decode (t_new == 1) or chunked prefill; with
// `advance` != 0 the positions then move on by that much (the decode step's cache advance);
// `shared_prefix` > 0 states that keys [0, shared_prefix) are the same in every row.
int kvcache_operator(const void *q, const void *k, const void *v, void *k_cache, void *v_cache,
                     const int32_t *cache_seqlens, int32_t *advance_seqlens, int advance,
                     int64_t shared_prefix, void *out, int64_t batch, int64_t t_new,
                     int64_t n_head, int64_t n_kv_head, int64_t head_dim, int64_t t_max,
                     int64_t cache_batch_stride, int64_t window, int dtype, void *workspace,
                     size_t workspace_bytes, hipStream_t stream) {
  if ((k == nullptr) != (v == nullptr))
    return fail(MCAMD_EINVAL, "flash_attn_with_kvcache: pass both k and v, or neither");
  AttnArgs a{q,     k,     v,      k_cache, v_cache,  cache_seqlens, out,
             batch, t_new, n_head, n_kv_head, head_dim, t_max,       cache_batch_stride,
             window, dtype, workspace, workspace_bytes, stream};
  int st = check_attn_shapes(a, t_new == 1);
  if (st != MCAMD_OK) return st;
  if (shared_prefix < 0 || shared_prefix > t_max)
    return fail(MCAMD_EINVAL, "flash_attn_with_kvcache: shared_prefix outside [0, t_max]");
  if (batch == 0) {
    clear_error();
    return MCAMD_OK;
  }
  if (t_new == 0) return launch_advance(advance_seqlens, batch, advance, stream);
  if (t_new == 1) {  // appends k/v itself, and advances the positions in its last pass
    a.advance_seqlens = advance ? advance_seqlens : nullptr;
    a.advance = advance;
    a.shared_prefix = shared_prefix;
    return launch_decode(a);
  }
  if (k) {
    AppendArgs ap{k,       v,        k_cache, v_cache, cache_seqlens,      batch, t_new,
                  n_kv_head, head_dim, t_max, cache_batch_stride, dtype, stream};
    st = launch_append(ap);
    if (st != MCAMD_OK) return st;
  }
  a.k_new = a.v_new = nullptr;
  st = launch_prefill(a);
  if (st != MCAMD_OK) return st;
  return launch_advance(advance_seqlens, batch, advance, stream);
}

}  // namespace

extern "C" int mcamd_flash_attn_varlen_with_kvcache(
    const void *q, const void *k, const void *v, void *k_cache, void *v_cache,
    int32_t *cache_seqlens, const int32_t *rows, const int32_t *cu_seqlens, void *out,
    int64_t n_seqs, int64_t max_seqlen, int64_t n_head, int64_t n_kv_head, int64_t head_dim,
    int64_t t_max, int64_t cache_batch_stride, int64_t window, int causal, int dtype, int advance,
    void *stream) {
  (void)causal;
  if ((k == nullptr) != (v == nullptr))
    return fail(MCAMD_EINVAL, "flash_attn_varlen_with_kvcache: pass both k and v, or neither");
  if (n_seqs > 0 && (!cu_seqlens || max_seqlen < 1))
    return fail(MCAMD_EINVAL,
                "flash_attn_varlen_with_kvcache: cu_seqlens and max_seqlen >= 1 are required");
  AttnArgs a{q,      k,          v,      k_cache,   v_cache,  cache_seqlens,      out,
             n_seqs, max_seqlen, n_head, n_kv_head, head_dim, t_max, cache_batch_stride,
             window, dtype,      nullptr, 0,        as_stream(stream)};
  a.rows = rows;
  a.cu = cu_seqlens;
  int st = check_attn_shapes(a, false);
  if (st != MCAMD_OK) return st;
  if (n_seqs == 0) {
    clear_error();
    return MCAMD_OK;
  }
  if (k) {
    AppendArgs ap{k,         v,        k_cache, v_cache, cache_seqlens,      n_seqs, max_seqlen,
                  n_kv_head, head_dim, t_max,   cache_batch_stride, dtype,   as_stream(stream)};
    ap.rows = rows;
    ap.cu = cu_seqlens;
    st = launch_append(ap);
    if (st != MCAMD_OK) return st;
  }
  a.k_new = a.v_new = nullptr;
  st = launch_prefill(a);
  if (st != MCAMD_OK) return st;
  if (!advance) return MCAMD_OK;
  return launch_advance_varlen(cache_seqlens, rows, cu_seqlens, n_seqs, as_stream(stream));
}

extern "C" int mcamd_flash_attn_with_kvcache(const void *q, const void *k, const void *v,
                                             void *k_cache, void *v_cache,
                                             const int32_t *cache_seqlens, void *out,
                                             int64_t batch, int64_t t_new, int64_t n_head,
                                             int64_t n_kv_head, int64_t head_dim, int64_t t_max,
                                             int64_t cache_batch_stride, int64_t window,
                                             int causal, int dtype, void *workspace,
                                             size_t workspace_bytes, void *stream) {
  (void)causal;
  return kvcache_operator(q, k, v, k_cache, v_cache, cache_seqlens, nullptr, 0, 0, out, batch,
                          t_new, n_head, n_kv_head, head_dim, t_max, cache_batch_stride, window,
                          dtype, workspace, workspace_bytes, as_stream(stream));
}

extern "C" int mcamd_flash_attn_with_kvcache_ex(
    const void *q, const void *k, const void *v, void *k_cache, void *v_cache,
    int32_t *cache_seqlens, void *out, int64_t batch, int64_t t_new, int64_t n_head,
    int64_t n_kv_head, int64_t head_dim, int64_t t_max, int64_t cache_batch_stride,
    int64_t window, int causal, int dtype, int32_t advance, int64_t shared_prefix,
    void *workspace, size_t workspace_bytes, void *stream) {
  (void)causal;
  return kvcache_operator(q, k, v, k_cache, v_cache, cache_seqlens, cache_seqlens, advance,
                          shared_prefix, out, batch, t_new, n_head, n_kv_head, head_dim, t_max,
                          cache_batch_stride, window, dtype, workspace, workspace_bytes,
                          as_stream(stream));
}
