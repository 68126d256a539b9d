// Internal launchers shared between the kernel translation units and the C ABI in capi.hip.
// Each returns an MCAMD_* status and sets the thread-local error message on failure.
#pragma once

#include "common.h"

namespace mcamd {

struct AppendArgs {
  const void *k, *v;
  void *k_cache, *v_cache;
  const int32_t *seqlens;
  int64_t batch, t_new, n_kv_head, head_dim, t_max, cache_batch_stride;
  int dtype;
  hipStream_t stream;
  // Varlen form (both optional): sequence b writes cache row rows[b] (b when null), and its new
  // tokens are [cu[b], cu[b + 1]) of k/v (t_new each, packed by sequence, when null); with cu,
  // t_new is the longest sequence's length.
  const int32_t *rows = nullptr;
  const int32_t *cu = nullptr;
};
int launch_append(const AppendArgs &a);

// seqlens[b] += advance for b < batch, one small kernel on `stream`.
int launch_advance(int32_t *seqlens, int64_t batch, int advance, hipStream_t stream);
// Varlen form: seqlens[rows[b]] += cu[b + 1] - cu[b] for b < n_seqs (rows null: row b).
int launch_advance_varlen(int32_t *seqlens, const int32_t *rows, const int32_t *cu,
                          int64_t n_seqs, hipStream_t stream);

struct AttnArgs {
  const void *q;
  const void *k_new, *v_new;  // decode only: the token at position cache_seqlens[b] is read from
                              // here instead of the cache (NULL = read it from the cache)
  const void *k_cache, *v_cache;
  const int32_t *seqlens;
  void *out;
  int64_t batch, t_new, n_head, n_kv_head, head_dim, t_max, cache_batch_stride, window;
  int dtype;
  void *workspace;
  size_t workspace_bytes;
  hipStream_t stream;
  // After the call has read the positions, cache_seqlens[b] += advance for every row (the
  // position advance of a decode step). The bf16 / head_dim 128 decode does it in its merge pass;
  // the other paths launch launch_advance after their kernels. advance 0: positions only read.
  int32_t *advance_seqlens = nullptr;
  int advance = 0;
  // Keys at positions [0, shared_prefix) hold the same K/V in every row (rows replicated from one
  // prompt): the bf16 / head_dim 128 decode reads them from row 0 for every row, so the rows'
  // repeated reads of those lines hit the caches. The other paths read each row's own copy.
  int64_t shared_prefix = 0;
  // Varlen prefill (launch_prefill only; both optional): sequence b uses cache row rows[b] (b when
  // null; cache_seqlens is indexed by the row) and its queries are tokens [cu[b], cu[b + 1]) of q
  // and out (t_new each when null; with cu, t_new is the longest sequence's length).
  const int32_t *rows = nullptr;
  const int32_t *cu = nullptr;
};
int launch_decode(const AttnArgs &a);
int launch_prefill(const AttnArgs &a);

// Split-K geometry of the decode path: keys per split and the number of splits a row can need.
constexpr int kDecodeSplitLen = 256;
int64_t decode_max_splits(int64_t t_max, int64_t window);

// Workspace of the decode path: scratch for the split partials (and the fused path's per-unit
// descriptors), written and read within one call; no contents are required on entry.
size_t decode_workspace_bytes(int64_t batch, int64_t n_head, int64_t n_kv_head, int64_t head_dim,
                              int64_t t_max, int64_t window);

// Units of the fused decode: one row's group of kDecodeUnitKv KV heads and kDecodeUnitQ query
// heads of each. A unit's split partials use the slot layout of kPartSlotBytes below.
constexpr int kDecodeUnitKv = 4;
constexpr int kDecodeUnitQ = 4;

// A split partial of a decode unit (the fused decode's segments and the shared prompt's key
// ranges): o[kv][q][128] as bf16 (each fp32 sum rounded once, to nearest even), then
// (m, l)[kv][q] as fp32 -- half the bytes of an all-fp32 slot, written by one launch and read
// back by the merge pass.
constexpr int kPartSlotOBytes = kDecodeUnitKv * kDecodeUnitQ * 128 * 2;
constexpr int kPartSlotBytes = kPartSlotOBytes + 2 * kDecodeUnitKv * kDecodeUnitQ * 4;

// Shared prompt prefix on the matrix cores: for every KV head, the queries of all rows against
// keys [0, prefix) of row 0, in n_split key ranges; each range's unnormalised (o, m, l) per
// (row, query head) goes to slot (unit * n_split + range), for the decode's merge pass to fold
// in.
#ifndef MCAMD_PREFIX_SPLITS
#define MCAMD_PREFIX_SPLITS 16
#endif
constexpr int kPrefixMaxSplits = MCAMD_PREFIX_SPLITS;
// Bytes of workspace past decode_workspace_bytes() for those partials (0 where the fused decode
// never takes the prefix on the matrix cores: such calls read row 0's keys in the streaming pass).
size_t decode_prefix_bytes(int64_t batch, int64_t n_head, int64_t n_kv_head, int64_t head_dim,
                           int64_t t_max, int64_t window);
// Whether the matrix-core kernel takes a (query heads, KV heads, T_max) geometry at all: at most
// 256 query heads per KV head (one workgroup's pairs) and one (row, KV head)'s cache addressable
// with 32-bit byte offsets.
bool prefill_mfma_geometry_ok(int64_t n_head, int64_t n_kv_head, int64_t t_max);

// The fused bf16 / head_dim 128 decode (append + split-K + merge in one launch).
bool decode_fused_supported(const AttnArgs &a);
int launch_decode_fused(const AttnArgs &a);
int64_t decode_fused_units(int64_t n_head, int64_t n_kv_head);
size_t decode_fused_partial_bytes(int64_t batch, int64_t n_head, int64_t n_kv_head,
                                  int64_t t_max, int64_t window);

// The general chunked prefill (any dtype, head_dim up to 512); it also serves single-token
// calls with head_dim above 256, past what the split-K decode kernel takes.
int launch_prefill_generic(const AttnArgs &a);

// The bf16 / head_dim 128 chunked prefill on the matrix cores.
bool prefill_mfma_supported(const AttnArgs &a);
int launch_prefill_mfma(const AttnArgs &a);

// Shape checks shared by every attention entry point.
int check_attn_shapes(const AttnArgs &a, bool need_workspace);

}  // namespace mcamd
