/*
 * modelcore_amd: C ABI of the MI355X (gfx950) KV-cache and cached-attention path.
 *
 * Every entry point takes plain device pointers, element counts and a hipStream_t passed as
 * `void *stream` (NULL = the null stream). Nothing here allocates device memory or synchronises
 * the host: work is enqueued on `stream` and the call returns. The library keeps two caches of
 * per-device facts, both safe to use from several threads: the compute-unit count of each device
 * (queried once, atomically published) and, for mcamd_flash_attn_with_kvcache_noalloc, the
 * address of its static scratch array on each device (looked up once, under a mutex).
 * Each function returns 0 on success or a negative MCAMD_E* code; mcamd_last_error() then
 * describes the failure (thread-local, valid until the next call on the same thread).
 *
 * Layouts (row-major, innermost dimension contiguous), matching the reference's cache object
 * and FA3-style operator (modelcore/cache.py:22-23, modelcore/kernels/flash_attn.py:313-322):
 *   k_cache, v_cache : (B, T_max, H_kv, D) per slot; `cache_batch_stride` (in elements) is the
 *                      distance between rows b and b+1 (T_max*H_kv*D for a contiguous slot view)
 *   q, out           : (B, T_new, H, D) contiguous
 *   k, v (new)       : (B, T_new, H_kv, D) contiguous
 *   cache_seqlens    : (B,) int32 on the device, the position of each row BEFORE these tokens
 * Query t of row b sits at position p = cache_seqlens[b] + t and attends keys col with
 * col <= p and (window < 0 or p - col <= window); softmax scale is 1/sqrt(D); query head h reads
 * KV head h / (H / H_kv).
 *
 * Attention takes head dims D with D * itemsize a multiple of 16, up to 512 (MCAMD_EUNSUPPORTED
 * past that, before anything is launched).
 *
 * A row whose positions fall outside [0, T_max) is not written by the append and gets NaN
 * attention output instead of an out-of-bounds access (the reference raises an index error there;
 * kernels cannot raise without a host sync).
 */
#ifndef MODELCORE_AMD_H
#define MODELCORE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of K/V/q/out. fp16 is absent, as in the reference (modelcore/runtime.py:22-23). */
enum { MCAMD_F32 = 0, MCAMD_BF16 = 1 };

/* Status codes. */
enum {
  MCAMD_OK = 0,
  MCAMD_EINVAL = -1,     /* bad argument: shape, dtype, alignment, null pointer */
  MCAMD_EUNSUPPORTED = -2, /* valid arguments this build has no kernel for */
  MCAMD_EWORKSPACE = -3, /* workspace missing or smaller than mcamd_attn_workspace_bytes() */
  MCAMD_ELAUNCH = -4     /* the HIP runtime refused a launch */
};

/* Version of this ABI; bumped on any signature change. */
int mcamd_abi_version(void);

/* Description of the last failure on this thread ("" after a success). */
const char *mcamd_last_error(void);

/*
 * KV append at per-row positions: for every row b and t < t_new,
 *   k_cache[b, cache_seqlens[b] + t] = k[b, t]   and likewise v_cache/v,
 * a bit-exact copy; nothing else in the caches changes.
 * Replaces the insert step of flash_attn_with_kvcache's fallback,
 * modelcore/kernels/flash_attn.py:336-346 (slice assignment, or index_put when ragged).
 */
int mcamd_kv_append(const void *k, const void *v, void *k_cache, void *v_cache,
                    const int32_t *cache_seqlens, int64_t batch, int64_t t_new,
                    int64_t n_kv_head, int64_t head_dim, int64_t t_max,
                    int64_t cache_batch_stride, int dtype, void *stream);

/*
 * Replication of one cache row into many: for every slot s, destination row r in
 * [dst_row_begin, dst_row_begin + n_rows) and position t < n_tokens,
 *   dst[s, r, t, :, :] = src[s, 0, t, :, :]        (bit-exact, K and V)
 * `src_k`/`src_v` point at slot 0, row 0 of the source; `row_elems` = H_kv * D; `dst_batch`
 * is the number of rows the destination has (the copy must fit in it). Strides are in elements.
 * Replaces KVCache.prefill's broadcast copy (modelcore/cache.py:84-85) and KVCache.prefill_row's
 * row copy (modelcore/cache.py:106-107).
 */
int mcamd_kv_replicate(const void *src_k, const void *src_v, void *dst_k, void *dst_v,
                       int64_t n_slots, int64_t src_slot_stride, int64_t dst_slot_stride,
                       int64_t dst_batch, int64_t dst_batch_stride, int64_t dst_row_begin,
                       int64_t n_rows, int64_t n_tokens, int64_t row_elems, int dtype,
                       void *stream);

/*
 * Bytes of scratch the attention entry points need for these sizes (split-K partials, and the
 * matrix-core partials of a shared prefix where mcamd_flash_attn_with_kvcache_ex could take
 * one). The caller allocates it (any 256-byte aligned device buffer) and passes it in.
 */
size_t mcamd_attn_workspace_bytes(int64_t batch, int64_t t_new, int64_t n_head,
                                  int64_t n_kv_head, int64_t head_dim, int64_t t_max,
                                  int64_t window);

/*
 * The cached-attention operator: optional append of (k, v) at cache_seqlens (k and v both
 * NULL = no append), then attention of q over the cache under the rules at the top of this
 * file. t_new == 1 runs split-K flash-decoding; t_new > 1 runs chunked prefill against the
 * cache prefix. cache_seqlens is read, never advanced. `causal` is accepted for signature
 * parity and ignored: the path is always causal.
 * Replaces flash_attn_with_kvcache (modelcore/kernels/flash_attn.py:306-366; the FA3 call at
 * :324-328 and the SDPA fallback at :330-366).
 */
int mcamd_flash_attn_with_kvcache(const void *q, const void *k, const void *v,
                                  void *k_cache, void *v_cache, const int32_t *cache_seqlens,
                                  void *out, int64_t batch, int64_t t_new, int64_t n_head,
                                  int64_t n_kv_head, int64_t head_dim, int64_t t_max,
                                  int64_t cache_batch_stride, int64_t window, int causal,
                                  int dtype, void *workspace, size_t workspace_bytes,
                                  void *stream);

/*
 * mcamd_flash_attn_with_kvcache with two extensions of the decode step, each off at 0.
 *  - advance: once the call has read cache_seqlens, cache_seqlens[b] += advance for every row b
 *    (rows outside the cache included), on the device, in stream order -- the step's position
 *    advance. For t_new == 1 with bf16 and head_dim 128 the add runs in the operator's own last
 *    pass (the merge, which does not read the positions), so the step needs no launch of its own
 *    for it; the other paths add one small kernel.
 *  - shared_prefix (0 <= shared_prefix <= t_max): the caller states that every row's K and V at
 *    positions [0, shared_prefix) are the same as row 0's (rows replicated from one prompt), and
 *    that every new token lands at or past shared_prefix. For t_new == 1 with bf16 and head_dim
 *    128, those keys are then taken from row 0 for every row. With no window, a prefix of at
 *    least 512 keys and at least 64 (row, query head) pairs per KV head, on the matrix cores:
 *    all rows' queries against row 0's prefix in key ranges, merged with the decode pass over
 *    each row's own keys -- the sums run in another order, so outputs agree with the call
 *    without it within bf16 rounding, not bit for bit (this needs the workspace size of
 *    mcamd_attn_workspace_bytes(); a smaller one that still covers the decode pass takes the
 *    other way). Otherwise the decode pass reads them from row 0 itself: the same values in the
 *    same order, so the same results bit for bit, with the rows' repeated reads of one row's
 *    lines served by the caches. Other paths read each row's own copy. A statement that does not
 *    hold gives rows row 0's keys below shared_prefix; on the matrix-core way, a row whose
 *    position lies below shared_prefix is moreover treated as outside the cache (NaN output, no
 *    append). The Python operator's checked mode raises for such a row before launching.
 * With both 0 this is exactly mcamd_flash_attn_with_kvcache; otherwise the cache contents are
 * bit-identical to that call's (followed by the separate advance) whenever the statement holds,
 * and the outputs as described above.
 * Replaces flash_attn_with_kvcache followed by KVCache.advance(advance) in a decode step
 * (modelcore/kernels/flash_attn.py:306-366, then modelcore/model.py:99-100 ->
 * modelcore/cache.py:62-73), after KVCache.prefill's replication (modelcore/cache.py:75-90).
 */
int mcamd_flash_attn_with_kvcache_ex(const void *q, const void *k, const void *v, void *k_cache,
                                     void *v_cache, int32_t *cache_seqlens, void *out,
                                     int64_t batch, int64_t t_new, int64_t n_head,
                                     int64_t n_kv_head, int64_t head_dim, int64_t t_max,
                                     int64_t cache_batch_stride, int64_t window, int causal,
                                     int dtype, int32_t advance, int64_t shared_prefix,
                                     void *workspace, size_t workspace_bytes, void *stream);

/*
 * mcamd_flash_attn_with_kvcache without the workspace arguments, for callers that cannot allocate
 * device memory (code under graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * It has no counterpart in the reference. Its scratch is a static device array of
 * MCAMD_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends), shared by every call on that
 * GPU: calls that overlap on one GPU race. Sizes whose decode partials need more scratch than that
 * (mcamd_attn_workspace_bytes() > MCAMD_NOALLOC_SCRATCH_BYTES) return MCAMD_EWORKSPACE. The
 * stream's device must be the current device. Otherwise identical to
 * mcamd_flash_attn_with_kvcache, with the same kernels and bit-identical results.
 */
#define MCAMD_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int mcamd_flash_attn_with_kvcache_noalloc(const void *q, const void *k, const void *v,
                                          void *k_cache, void *v_cache,
                                          const int32_t *cache_seqlens, void *out, int64_t batch,
                                          int64_t t_new, int64_t n_head, int64_t n_kv_head,
                                          int64_t head_dim, int64_t t_max,
                                          int64_t cache_batch_stride, int64_t window, int causal,
                                          int dtype, void *stream);

/*
 * Attention only (no append), one query token per row: the decode half of
 * mcamd_flash_attn_with_kvcache for t_new == 1 (modelcore/kernels/flash_attn.py:348-366 with
 * T_new == 1). Exposed separately so the append and the attention can be timed apart.
 */
int mcamd_decode_attention(const void *q, const void *k_cache, const void *v_cache,
                           const int32_t *cache_seqlens, void *out, int64_t batch,
                           int64_t n_head, int64_t n_kv_head, int64_t head_dim, int64_t t_max,
                           int64_t cache_batch_stride, int64_t window, int dtype,
                           void *workspace, size_t workspace_bytes, void *stream);

/*
 * Attention only (no append), t_new >= 1 query tokens per row against the cache prefix: the
 * chunked-prefill half of mcamd_flash_attn_with_kvcache (modelcore/kernels/flash_attn.py:226-244
 * and :362-364, T_new > 1).
 */
int mcamd_prefill_attention(const void *q, const void *k_cache, const void *v_cache,
                            const int32_t *cache_seqlens, void *out, int64_t batch,
                            int64_t t_new, int64_t n_head, int64_t n_kv_head, int64_t head_dim,
                            int64_t t_max, int64_t cache_batch_stride, int64_t window,
                            int dtype, void *stream);

/*
 * Varlen chunked prefill: n_seqs sequences of different lengths, each appended and attended in
 * its own cache row, with no padding. Sequence b is tokens [cu_seqlens[b], cu_seqlens[b + 1]) of
 * the packed q (total, H, D), k and v (total, H_kv, D) and out (total, H, D), cu_seqlens being
 * n_seqs + 1 ascending int32 offsets on the device (cu_seqlens[0] = 0); max_seqlen (>= 1) is the
 * longest sequence's length, which sizes the grids. Sequence b uses cache row rows[b] (rows: n_seqs
 * distinct int32 row indices on the device, or NULL for row b; not checked on the host); its query
 * t sits at position cache_seqlens[rows[b]] + t, with the same key visibility as
 * mcamd_flash_attn_with_kvcache. k and v (both, or neither) are appended bit-exactly at those
 * positions first. With advance != 0, cache_seqlens[rows[b]] then grows by the sequence's length.
 * A sequence whose positions fall outside [0, t_max) gets NaN output, and its append drops the
 * positions past the cache (as mcamd_kv_append does).
 * Replaces the reference's multi-prompt prefill -- each prompt prefilled alone into a batch-1
 * cache, then copied into its row (modelcore/generate.py:67-80 -> KVCache.prefill_row,
 * modelcore/cache.py:92-119) -- with one batched call per layer that writes every prompt's K/V in
 * place; attention per sequence as modelcore/kernels/flash_attn.py:226-244, 362-364.
 */
int mcamd_flash_attn_varlen_with_kvcache(const void *q, const void *k, const void *v,
                                         void *k_cache, void *v_cache, int32_t *cache_seqlens,
                                         const int32_t *rows, const int32_t *cu_seqlens, void *out,
                                         int64_t n_seqs, int64_t max_seqlen, int64_t n_head,
                                         int64_t n_kv_head, int64_t head_dim, int64_t t_max,
                                         int64_t cache_batch_stride, int64_t window, int causal,
                                         int dtype, int advance, void *stream);

/*
 * Next-token sampling on the device, one token per row of `logits` ((batch, vocab) fp32, rows
 * `row_stride` elements apart; 0 = every row reads the same logits): temperature 0 takes the
 * argmax (lowest index on ties); otherwise the Gumbel-max draw from softmax(logits / temperature)
 * with Philox4x32-10 noise keyed by the row's 64-bit `seeds[b]` at counter offsets[b], which the
 * call then advances by one (device side, no host sync). 0 < top_k < vocab restricts the draw to
 * the top_k largest logits of the row (ties at the k-th value kept lowest index first); top_k <= 0
 * or >= vocab draws from all of them. Writes int64 token ids to out[b].
 * Replaces sample_next_token's softmax + torch.multinomial, and its top_k branch (torch.topk, then
 * the draw over the kept logits) (modelcore/generate.py:18-34); the per-row counter stream stands
 * in for its single torch.Generator, so a row's draws do not depend on the batch it is decoded in.
 */
int mcamd_sample_tokens(const float *logits, int64_t batch, int64_t vocab, int64_t row_stride,
                        float temperature, int64_t top_k, const uint64_t *seeds, int64_t *offsets,
                        int64_t *out, void *stream);

/*
 * The step before the operator, fused: RoPE at each token's position p = cache_seqlens[b] + t,
 * RMS-norm over head_dim (eps added to the mean square, fp32 arithmetic), and `scale`, applied to
 * q (written to q_out, (batch, t_new, n_head, head_dim) contiguous) and to k, which is then
 * appended with v. q, k, v are (batch, t_new, heads, head_dim) with heads contiguous and tokens
 * `*_token_stride` elements apart (the views of a fused QKV projection); k is appended with v
 * at p as mcamd_kv_append does. `cos`/`sin` are the rotary tables, (n_pos, head_dim / 2) in the
 * storage dtype. k = v = NULL transforms q only (k_cache/v_cache unused). Each rotation product
 * and sum is rounded to the storage dtype like the separate torch ops; only the order of the
 * fp32 sum of squares differs from them (results within one unit in the last place).
 * Replaces, in modelcore/components/attention.py:143-150 (producer layers) and :155-157
 * (KV-sharing consumers): RotaryEmbedding.forward/apply_to_q (modelcore/components/rotary.py:
 * 69-81 -> rope.py:4-12), the QK RMSNorm (modelcore/components/norm.py:43-44), the two x1.2
 * multiplies, and the append half of flash_attn_with_kvcache (modelcore/kernels/flash_attn.py:
 * 336-346). Positions come from cache_seqlens on the device: no host sync.
 */
int mcamd_qk_rope_norm_append(const void *q, int64_t q_token_stride, const void *k,
                              int64_t k_token_stride, const void *v, int64_t v_token_stride,
                              const void *cos, const void *sin, int64_t n_pos, void *k_cache,
                              void *v_cache,
                              const int32_t *cache_seqlens, void *q_out, int64_t batch,
                              int64_t t_new, int64_t n_head, int64_t n_kv_head, int64_t head_dim,
                              int64_t t_max, int64_t cache_batch_stride, float eps, float scale,
                              int dtype, void *stream);

/*
 * mcamd_qk_rope_norm_append for bf16, reading q, k, v from the unsummed K-split partials of the
 * stacked QKV projection (mcamd_linear_bf16_partials of x with [W_q; W_k; W_v]): `part` is
 * (splits, batch * t_new, part_token_stride) fp32, q at columns [0, H D), k at [H D, (H + H_kv) D),
 * v after it; each value is the in-order sum of the splits rounded to bf16, which is what
 * mcamd_linear_bf16 outputs. with_kv = 0: q only (k_cache, v_cache unused). Saves the projection's
 * separate reduce pass; otherwise as mcamd_qk_rope_norm_append.
 */
int mcamd_qk_rope_norm_append_partials(const float *part, int64_t splits,
                                       int64_t part_token_stride, const void *cos,
                                       const void *sin, int64_t n_pos, void *k_cache,
                                       void *v_cache, const int32_t *cache_seqlens, void *q_out,
                                       int64_t batch, int64_t t_new, int64_t n_head,
                                       int64_t n_kv_head, int64_t head_dim, int64_t t_max,
                                       int64_t cache_batch_stride, float eps, float scale,
                                       int with_kv, void *stream);

/*
 * y = x . W^T for decode-sized batches: x (m, k) bf16 rows `ldx` elements apart, m <= 64; W
 * (n, k) bf16 contiguous (the nn.Linear weight layout); y (m, n) bf16 rows `ldy` apart; fp32
 * accumulation. n must be a multiple of 64 and k of 128 * k_splits. With k_splits > 1 the K
 * range is split across workgroups and the partial products are summed in a fixed order by a
 * second kernel (deterministic), using `workspace` of mcamd_linear_bf16_workspace_bytes() bytes.
 * Replaces F.linear in Linear.forward (modelcore/components/linear.py:13-14) for the projections
 * of a decode step, where reading the weights once from HBM is the whole cost.
 */
size_t mcamd_linear_bf16_workspace_bytes(int64_t m, int64_t n, int64_t k_splits);
int mcamd_linear_bf16(const void *x, int64_t ldx, const void *w, void *y, int64_t ldy, int64_t m,
                      int64_t n, int64_t k, int64_t k_splits, void *workspace,
                      size_t workspace_bytes, void *stream);

/*
 * The gated MLP's first half at decode sizes: with W = [W_gate; W_up] interleaved in blocks of 64
 * rows (rows 128 b .. 128 b + 63 = gate rows 64 b .. 64 b + 63, the next 64 = the up rows of the
 * same units; W is (2 hidden, k)), writes h (m, hidden) bf16, rows `ldh` apart:
 *   h[r][j] = bf16(bf16(act(g)) * u),  g = bf16(x[r] . W_gate[j]),  u = bf16(x[r] . W_up[j])
 * in fp32 arithmetic, i.e. torch's `act(gate(x)) * up(x)` on bf16 tensors. act = MCAMD_ACT_SILU
 * (x / (1 + e^-x)); hidden a multiple of 64, k of 128, m <= 64. w_tiled = 1: W is stored as
 * (2 hidden / 64, k / 128, 64, 128) contiguous blocks (block [g][s] = rows 64 g .. 64 g + 63,
 * columns 128 s .. 128 s + 127, row-major), so that the weight stream reads whole 1 KB runs;
 * 0: row-major (2 hidden, k). Replaces GatedMLP.forward's gate_proj, up_proj and the activation
 * product (modelcore/components/mlp.py:89-90) before down_proj.
 */
enum { MCAMD_ACT_SILU = 0 };
int mcamd_linear_bf16_gated(const void *x, int64_t ldx, const void *w, void *h, int64_t ldh,
                            int64_t m, int64_t hidden, int64_t k, int act, int w_tiled,
                            void *stream);

/*
 * mcamd_linear_bf16 without the sum: the K-split partial products, written to `part` as
 * (k_splits, m, n) fp32 (k_splits = 1 included), for a consumer that sums them itself in the
 * same order (mcamd_residual_rmsnorm). Same shape rules as mcamd_linear_bf16; part 16-byte
 * aligned, k_splits * m * n floats. Replaces the same F.linear call sites (c_proj and down_proj
 * in the reference, modelcore/components/attention.py:183, modelcore/components/mlp.py:90), with
 * the reduction left to the fused residual step below.
 */
int mcamd_linear_bf16_partials(const void *x, int64_t ldx, const void *w, float *part, int64_t m,
                               int64_t n, int64_t k, int64_t k_splits, void *stream);

/*
 * The residual update and the next RMS-norm, fused, for (m, n) bf16 rows (contiguous, n a
 * multiple of 8):
 *   y     = bf16(sum_s part[s])  (part: (splits, m, n) fp32, summed in order s = 0, 1, ...),
 *           or y given in bf16 (part = NULL)
 *   x_out = bf16(x + y)
 *   h_out = bf16(x_out * rsqrt(mean(x_out^2) + eps))   (fp32 arithmetic)
 * x_out may be x itself (an in-place update of the residual stream); h_out is a buffer of its own.
 * Replaces, in a block (modelcore/components/block.py:54-60), the residual add `x + f(norm(x))`
 * and the RMSNorm that follows it (modelcore/components/norm.py:43-44), plus the split-K sum of
 * the projection that produced f.
 */
int mcamd_residual_rmsnorm(const void *x, const float *part, int64_t splits, const void *y,
                           void *x_out, void *h_out, int64_t m, int64_t n, float eps,
                           void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MODELCORE_AMD_H */
