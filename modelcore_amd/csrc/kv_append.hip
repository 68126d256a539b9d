// KV append: scatter of the new tokens' K/V rows into the cache at per-row positions.
//
// Semantics follow modelcore/kernels/flash_attn.py:336-346: for each row b and t < t_new,
// cache[b, cache_seqlens[b] + t] = new[b, t]. One token's K (or V) for all KV heads is a
// contiguous H_kv*D run in both the source (B, T_new, H_kv, D) and the cache
// (B, T_max, H_kv, D), so the append is a copy of B*T_new contiguous runs. The copy is bit-exact:
// no arithmetic touches the data.
//
// Grid: (blocks over one row's T_new runs, 2 (K, V), B rows, 65535 per launch). A workgroup
// reads cache_seqlens[b] once (a uniform load) and moves kUnroll * 256 units of 16 bytes (or 4/2
// when a run is not 16-byte divisible) of row b; each thread issues its kUnroll loads before its
// stores. Unit -> (token, offset) is a shift and a mask when a run holds a power of two of units,
// a division otherwise. For a 512-token chunk of 8 rows x 8 KV heads x 128 bf16 (16.8 MB in,
// 16.8 MB out) two units per thread at 256 threads took 7.41 us; one unit 7.92, four 8.26, 512 or
// 1024 threads 7.7-8.6, non-temporal stores 9.2, hipMemcpyAsync of the same bytes 9.2 us, and a
// grid-stride loop of one unit per thread with per-unit divisions 8.6-8.7 us.
#include <algorithm>

#include "kernels.h"

namespace mcamd {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kUnroll = 2;

// Sequence b = b_first + blockIdx.z goes to cache row rows[b] (b when rows is null); its new
// tokens are t_new consecutive tokens from token b * t_new of k/v, or, with cu (the varlen form:
// sequences of different lengths packed one after another), tokens [cu[b], cu[b + 1]).
template <class U, bool POW2>
__global__ __launch_bounds__(kThreads) void kv_append_kernel(
    const U *__restrict__ k, const U *__restrict__ v, U *__restrict__ k_cache,
    U *__restrict__ v_cache, const int32_t *__restrict__ seqlens, const int32_t *__restrict__ rows,
    const int32_t *__restrict__ cu, int b_first, int t_new, int units_per_row, int upr_shift,
    int64_t t_max, int64_t cache_b_units) {
  const int b = b_first + int(blockIdx.z);
  const int row = rows ? rows[b] : b;
  const int64_t tok0 = cu ? int64_t(cu[b]) : int64_t(b) * t_new;
  const int t_b = cu ? cu[b + 1] - cu[b] : t_new;
  const U *src = (blockIdx.y == 0 ? k : v) + tok0 * units_per_row;
  U *dst = (blockIdx.y == 0 ? k_cache : v_cache) + int64_t(row) * cache_b_units;
  const int64_t s0 = seqlens[row];
  const int row_units = t_b * units_per_row;  // this row's units (fits 32 bits: checked)
  const int base = blockIdx.x * (kThreads * kUnroll);
  if (base >= row_units) return;  // varlen: a shorter sequence than the grid's longest
  const int first = base + threadIdx.x;
  const int last = std::min(base + kThreads * kUnroll, row_units) - 1;  // uniform
  const int t_first = POW2 ? base >> upr_shift : base / units_per_row;
  const int t_last = POW2 ? last >> upr_shift : last / units_per_row;
  U val[kUnroll];
  if (last == base + kThreads * kUnroll - 1 && s0 + t_first >= 0 && s0 + t_last < t_max) {
    // Whole block in range (the common case): no per-unit checks, all loads before the stores.
#pragma unroll
    for (int j = 0; j < kUnroll; ++j) val[j] = src[first + j * kThreads];
#pragma unroll
    for (int j = 0; j < kUnroll; ++j) {
      const int i = first + j * kThreads;
      const int t = POW2 ? i >> upr_shift : i / units_per_row;
      const int u = POW2 ? i & (units_per_row - 1) : i - t * units_per_row;
      dst[(s0 + t) * units_per_row + u] = val[j];
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < kUnroll; ++j) {
    const int i = first + j * kThreads;
    if (i > last) continue;
    const int t = POW2 ? i >> upr_shift : i / units_per_row;
    const int u = POW2 ? i & (units_per_row - 1) : i - t * units_per_row;
    const int64_t pos = s0 + t;
    if (pos < 0 || pos >= t_max) continue;  // out-of-range rows are left untouched
    dst[pos * units_per_row + u] = src[i];
  }
}

template <class U>
int run(const AppendArgs &a, int64_t row_bytes) {
  const int64_t upr = row_bytes / int64_t(sizeof(U));
  const int64_t elem = a.dtype == MCAMD_F32 ? 4 : 2;
  const int64_t cb_units = a.cache_batch_stride * elem / int64_t(sizeof(U));
  if (a.batch == 0 || a.t_new == 0) {
    clear_error();
    return MCAMD_OK;
  }
  // The kernel's int unit indices reach the row's unit count plus one block's reach.
  if (a.t_new * upr > (int64_t(1) << 31) - 1 - int64_t(kThreads) * kUnroll)
    return fail(MCAMD_EUNSUPPORTED, "kv_append: too many units in one row's new tokens for 32-bit "
                                    "indices");
  const int64_t per_block = int64_t(kThreads) * kUnroll;
  // Varlen: t_new is the longest sequence's token count (sizes the grid).
  const unsigned blocks = unsigned((a.t_new * upr + per_block - 1) / per_block);
  int shift = 0;
  while ((int64_t(1) << shift) < upr) ++shift;
  const bool pow2 = (int64_t(1) << shift) == upr;
  // Rows go in the grid's z dimension, at most 65535 per launch.
  constexpr int64_t kRowsPerLaunch = 65535;
  for (int64_t b0 = 0; b0 < a.batch; b0 += kRowsPerLaunch) {
    const int64_t n = std::min(kRowsPerLaunch, a.batch - b0);
    const dim3 grid(blocks, 2, unsigned(n));
    auto go = [&](auto kernel) {
      hipLaunchKernelGGL(kernel, grid, dim3(kThreads), 0, a.stream, static_cast<const U *>(a.k),
                         static_cast<const U *>(a.v), static_cast<U *>(a.k_cache),
                         static_cast<U *>(a.v_cache), a.seqlens, a.rows, a.cu, int(b0),
                         int(a.t_new), int(upr), shift, a.t_max, cb_units);
    };
    if (pow2)
      go(kv_append_kernel<U, true>);
    else
      go(kv_append_kernel<U, false>);
  }
  return launch_status("kv_append");
}

// Position advance of a decode step (modelcore/cache.py:62-73, cache_seqlens += num_tokens), for
// the operator paths whose kernels have no later pass to fold it into.
__global__ __launch_bounds__(256) void advance_kernel(int32_t *seqlens, int batch, int by) {
  for (int b = blockIdx.x * 256 + threadIdx.x; b < batch; b += gridDim.x * 256) seqlens[b] += by;
}

__global__ __launch_bounds__(256) void advance_varlen_kernel(int32_t *seqlens,
                                                             const int32_t *rows,
                                                             const int32_t *cu, int n) {
  for (int b = blockIdx.x * 256 + threadIdx.x; b < n; b += gridDim.x * 256)
    seqlens[rows ? rows[b] : b] += cu[b + 1] - cu[b];
}

}  // namespace

int launch_advance_varlen(int32_t *seqlens, const int32_t *rows, const int32_t *cu,
                          int64_t n_seqs, hipStream_t stream) {
  if (n_seqs <= 0) {
    clear_error();
    return MCAMD_OK;
  }
  if (!seqlens || !cu) return fail(MCAMD_EINVAL, "advance: null cache_seqlens or cu_seqlens");
  const int blocks = int(std::min<int64_t>((n_seqs + 255) / 256, 256));
  hipLaunchKernelGGL(advance_varlen_kernel, dim3(blocks), dim3(256), 0, stream, seqlens, rows,
                     cu, int(n_seqs));
  return launch_status("advance_varlen");
}

int launch_advance(int32_t *seqlens, int64_t batch, int advance, hipStream_t stream) {
  if (batch <= 0 || advance == 0) {
    clear_error();
    return MCAMD_OK;
  }
  if (!seqlens) return fail(MCAMD_EINVAL, "advance: null cache_seqlens");
  const int blocks = int(std::min<int64_t>((batch + 255) / 256, 256));
  hipLaunchKernelGGL(advance_kernel, dim3(blocks), dim3(256), 0, stream, seqlens, int(batch),
                     advance);
  return launch_status("advance");
}

int launch_append(const AppendArgs &a) {
  if (a.dtype != MCAMD_F32 && a.dtype != MCAMD_BF16)
    return fail(MCAMD_EINVAL, "kv_append: dtype must be MCAMD_F32 or MCAMD_BF16");
  if (a.batch < 0 || a.t_new < 0 || a.n_kv_head <= 0 || a.head_dim <= 0 || a.t_max <= 0)
    return fail(MCAMD_EINVAL, "kv_append: sizes must be positive (batch, t_new may be 0)");
  if (!a.k || !a.v || !a.k_cache || !a.v_cache || !a.seqlens)
    return fail(MCAMD_EINVAL, "kv_append: null pointer");
  if (a.cache_batch_stride < a.t_max * a.n_kv_head * a.head_dim)
    return fail(MCAMD_EINVAL, "kv_append: cache_batch_stride smaller than T_max*H_kv*D");
  const int64_t elem = a.dtype == MCAMD_F32 ? 4 : 2;
  const int64_t row_bytes = a.n_kv_head * a.head_dim * elem;
  const int64_t cb_bytes = a.cache_batch_stride * elem;
  auto ok16 = [&](const void *p) { return aligned(p, 16); };
  if (row_bytes % 16 == 0 && cb_bytes % 16 == 0 && ok16(a.k) && ok16(a.v) && ok16(a.k_cache) &&
      ok16(a.v_cache))
    return run<u32x4>(a, row_bytes);
  auto ok4 = [&](const void *p) { return aligned(p, 4); };
  if (row_bytes % 4 == 0 && cb_bytes % 4 == 0 && ok4(a.k) && ok4(a.v) && ok4(a.k_cache) &&
      ok4(a.v_cache))
    return run<uint32_t>(a, row_bytes);
  return run<uint16_t>(a, row_bytes);
}

}  // namespace mcamd
