// The cached-attention operator without a caller-supplied workspace, for callers that cannot
// allocate device memory (code under graph capture, tight serving loops, harnesses that forbid
// hipMalloc). Its scratch is a file-scope device array of kScratchBytes per GPU, held for the
// life of the process; the entry point itself calls no allocating routine.
//
// In host code `scratch` names a host-side stand-in, not the device array: its device address is
// looked up once per device with hipGetSymbolAddress (with that device current) and only that
// address is handed to the kernels. Every call on a device shares that device's array and leaves
// its partials there: calls that overlap on one GPU (two streams at once) race.
#include "kernels.h"

#include <mutex>
#include <string>

namespace mcamd {
namespace {

constexpr size_t kScratchBytes = MCAMD_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

__device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on the first call there).
int scratch_on_current_device(void **ptr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return fail(MCAMD_ELAUNCH, std::string("noalloc: hipGetDevice: ") + hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(MCAMD_EUNSUPPORTED, "noalloc: device index beyond " + std::to_string(kMaxDevices));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(MCAMD_ELAUNCH, std::string("noalloc: hipGetSymbolAddress(scratch): ") +
                                     hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return MCAMD_OK;
}

}  // namespace
}  // namespace mcamd

using namespace mcamd;

extern "C" int mcamd_flash_attn_with_kvcache_noalloc(
    const void *q, const void *k, const void *v, void *k_cache, void *v_cache,
    const int32_t *cache_seqlens, void *out, int64_t batch, int64_t t_new, int64_t n_head,
    int64_t n_kv_head, int64_t head_dim, int64_t t_max, int64_t cache_batch_stride,
    int64_t window, int causal, int dtype, void *stream) {
  size_t need = 0;
  if (t_new == 1 && batch > 0 && n_kv_head > 0 && n_head >= n_kv_head && head_dim > 0 && t_max > 0)
    need = decode_workspace_bytes(batch, n_head, n_kv_head, head_dim, t_max, window);
  if (need > kScratchBytes)
    return fail(MCAMD_EWORKSPACE, "flash_attn_with_kvcache_noalloc: these sizes need " +
                                      std::to_string(need) + " bytes of scratch, more than the " +
                                      std::to_string(kScratchBytes) +
                                      " of the static array; use mcamd_flash_attn_with_kvcache "
                                      "with a workspace");
  void *ptr = nullptr;
  if (need > 0) {
    const int st = scratch_on_current_device(&ptr);
    if (st != MCAMD_OK) return st;
  }
  return mcamd_flash_attn_with_kvcache(q, k, v, k_cache, v_cache, cache_seqlens, out, batch, t_new,
                                       n_head, n_kv_head, head_dim, t_max, cache_batch_stride,
                                       window, causal, dtype, ptr, need > 0 ? kScratchBytes : 0,
                                       stream);
}
