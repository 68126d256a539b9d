// KV append: scatter of the new tokens' K/V rows into the cache at per-row positions.
//
// Semantics follow modelcore/kernels/flash_attn.py:336-346: for each row b and t < t_new,
// cache[b, cache_seqlens[b] + t] = new[b, t]. One token's K (or V) for all KV heads is a
// contiguous H_kv*D run in both the source (B, T_new, H_kv, D) and the cache
// (B, T_max, H_kv, D), so the append is a copy of B*T_new contiguous runs. Each thread moves one
// 16-byte unit (or 4/2 bytes when a run is not 16-byte divisible), so a wave writes 1 KiB of one
// run per instruction. The copy is bit-exact: no arithmetic touches the data.
#include "kernels.h"

namespace mcamd {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <class U>
__global__ __launch_bounds__(256) void kv_append_kernel(const U *__restrict__ k,
                                                        const U *__restrict__ v,
                                                        U *__restrict__ k_cache,
                                                        U *__restrict__ v_cache,
                                                        const int32_t *__restrict__ seqlens,
                                                        int64_t t_new, int64_t units_per_row,
                                                        int64_t t_max, int64_t cache_b_units,
                                                        int64_t total_units) {
  const U *src = blockIdx.y == 0 ? k : v;
  U *dst = blockIdx.y == 0 ? k_cache : v_cache;
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total_units; i += stride) {
    const int64_t row = i / units_per_row;
    const int64_t u = i - row * units_per_row;
    const int64_t b = row / t_new;
    const int64_t t = row - b * t_new;
    const int64_t pos = int64_t(seqlens[b]) + t;
    if (pos < 0 || pos >= t_max) continue;  // out-of-range rows are left untouched
    dst[b * cache_b_units + pos * units_per_row + u] = src[i];
  }
}

template <class U>
int run(const AppendArgs &a, int64_t row_bytes) {
  const int64_t upr = row_bytes / int64_t(sizeof(U));
  const int64_t elem = a.dtype == MCAMD_F32 ? 4 : 2;
  const int64_t cb_units = a.cache_batch_stride * elem / int64_t(sizeof(U));
  const int64_t total = a.batch * a.t_new * upr;
  if (total == 0) {
    clear_error();
    return MCAMD_OK;
  }
  const int threads = 256;
  int64_t blocks = (total + threads - 1) / threads;
  if (blocks > 65535 * 8) blocks = 65535 * 8;
  hipLaunchKernelGGL(kv_append_kernel<U>, dim3(unsigned(blocks), 2), dim3(threads), 0, a.stream,
                     static_cast<const U *>(a.k), static_cast<const U *>(a.v),
                     static_cast<U *>(a.k_cache), static_cast<U *>(a.v_cache), a.seqlens, a.t_new,
                     upr, a.t_max, cb_units, total);
  return launch_status("kv_append");
}

}  // namespace

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
