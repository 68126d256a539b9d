// KV replication: copy row 0 of a source cache into rows [row_begin, row_begin + n_rows) of a
// destination cache, for every slot, K and V.
//
// Semantics follow KVCache.prefill (modelcore/cache.py:84-85, a broadcast over all rows) and
// KVCache.prefill_row (modelcore/cache.py:106-107, one row). The source run of a slot, the first
// n_tokens positions of row 0, is H_kv*D*n_tokens contiguous elements; so is its image in each
// destination row. Each thread loads one 16-byte unit of the source once and stores it into every
// destination row with non-temporal stores: the source is read from HBM once, the n_rows copies
// stream out without displacing the source from L2. Bit-exact: no arithmetic touches the data.
#include "kernels.h"

namespace mcamd {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <class U>
__global__ __launch_bounds__(256) void kv_replicate_kernel(
    const U *__restrict__ src_k, const U *__restrict__ src_v, U *__restrict__ dst_k,
    U *__restrict__ dst_v, int64_t src_slot_units, int64_t dst_slot_units,
    int64_t dst_batch_units, int64_t row_begin, int64_t n_rows, int64_t units_per_slot) {
  const int64_t slot = blockIdx.y;
  const U *src = (blockIdx.z == 0 ? src_k : src_v) + slot * src_slot_units;
  U *dst = (blockIdx.z == 0 ? dst_k : dst_v) + slot * dst_slot_units + row_begin * dst_batch_units;
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < units_per_slot;
       i += stride) {
    const U x = src[i];
    U *d = dst + i;
    for (int64_t r = 0; r < n_rows; ++r) __builtin_nontemporal_store(x, d + r * dst_batch_units);
  }
}

template <class U>
int run(const void *src_k, const void *src_v, void *dst_k, void *dst_v, int64_t n_slots,
        int64_t src_slot_stride, int64_t dst_slot_stride, int64_t dst_batch_stride,
        int64_t row_begin, int64_t n_rows, int64_t n_tokens, int64_t row_elems, int64_t elem,
        hipStream_t stream) {
  const int64_t us = int64_t(sizeof(U));
  const int64_t units = n_tokens * row_elems * elem / us;
  if (units == 0 || n_rows == 0 || n_slots == 0) {
    clear_error();
    return MCAMD_OK;
  }
  const int threads = 256;
  int64_t blocks = (units + threads - 1) / threads;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(kv_replicate_kernel<U>, dim3(unsigned(blocks), unsigned(n_slots), 2),
                     dim3(threads), 0, stream, static_cast<const U *>(src_k),
                     static_cast<const U *>(src_v), static_cast<U *>(dst_k),
                     static_cast<U *>(dst_v), src_slot_stride * elem / us,
                     dst_slot_stride * elem / us, dst_batch_stride * elem / us, row_begin,
                     n_rows, units);
  return launch_status("kv_replicate");
}

}  // namespace
}  // namespace mcamd

using namespace mcamd;

extern "C" int mcamd_kv_replicate(const void *src_k, const void *src_v, void *dst_k,
                                  void *dst_v, int64_t n_slots, int64_t src_slot_stride,
                                  int64_t dst_slot_stride, int64_t dst_batch,
                                  int64_t dst_batch_stride, int64_t dst_row_begin, int64_t n_rows,
                                  int64_t n_tokens, int64_t row_elems, int dtype, void *stream) {
  if (dtype != MCAMD_F32 && dtype != MCAMD_BF16)
    return fail(MCAMD_EINVAL, "kv_replicate: dtype must be MCAMD_F32 or MCAMD_BF16");
  if (n_slots < 0 || n_rows < 0 || n_tokens < 0 || row_elems <= 0 || dst_row_begin < 0)
    return fail(MCAMD_EINVAL, "kv_replicate: negative size");
  if (n_slots > 65535) return fail(MCAMD_EUNSUPPORTED, "kv_replicate: more than 65535 slots");
  if (n_slots > 0 && n_rows > 0 && n_tokens > 0 && (!src_k || !src_v || !dst_k || !dst_v))
    return fail(MCAMD_EINVAL, "kv_replicate: null pointer");
  if (dst_row_begin + n_rows > dst_batch)
    return fail(MCAMD_EINVAL, "kv_replicate: destination rows past the destination batch");
  if (dst_batch_stride < n_tokens * row_elems)
    return fail(MCAMD_EINVAL, "kv_replicate: destination row smaller than the copied run");
  if (n_slots > 1 && (src_slot_stride < n_tokens * row_elems ||
                      dst_slot_stride < dst_batch * dst_batch_stride))
    return fail(MCAMD_EINVAL, "kv_replicate: slot stride smaller than one slot");
  const int64_t elem = dtype == MCAMD_F32 ? 4 : 2;
  const int64_t run_bytes = n_tokens * row_elems * elem;
  auto fits = [&](int64_t a) {
    return run_bytes % a == 0 && (src_slot_stride * elem) % a == 0 &&
           (dst_slot_stride * elem) % a == 0 && (dst_batch_stride * elem) % a == 0 &&
           aligned(src_k, a) && aligned(src_v, a) && aligned(dst_k, a) && aligned(dst_v, a);
  };
  hipStream_t s = as_stream(stream);
  if (fits(16))
    return run<u32x4>(src_k, src_v, dst_k, dst_v, n_slots, src_slot_stride, dst_slot_stride,
                      dst_batch_stride, dst_row_begin, n_rows, n_tokens, row_elems, elem, s);
  if (fits(4))
    return run<uint32_t>(src_k, src_v, dst_k, dst_v, n_slots, src_slot_stride, dst_slot_stride,
                         dst_batch_stride, dst_row_begin, n_rows, n_tokens, row_elems, elem, s);
  return run<uint16_t>(src_k, src_v, dst_k, dst_v, n_slots, src_slot_stride, dst_slot_stride,
                       dst_batch_stride, dst_row_begin, n_rows, n_tokens, row_elems, elem, s);
}
