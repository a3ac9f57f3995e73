// fk_paged_decode_noalloc: fk_paged_decode for callers that cannot allocate
// (code under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc).  It has no counterpart in the reference.
//
// The split-context workspace is `scratch`, a file-scope device array that each
// GPU holds from module load until the process ends.  In host code the array's
// name is only a stand-in, so its device address is resolved with
// hipGetSymbolAddress on the first call on each device (with that device
// current) and kept per device; only that address is passed to the kernels
// (through fk_paged_decode's workspace argument).  Every call on a device shares
// the array, and it keeps the last call's contents: calls that overlap on one
// device (concurrent streams or threads) race on it.  Nothing in the workspace
// must start at zero -- the main kernel writes the schedule and every partial
// row the merge kernel reads -- so no clearing is needed between calls.
#include <stdio.h>

#include <mutex>

#include "fk_common.h"

namespace fk {
namespace {

static __device__ __align__(256) uint8_t scratch[FK_PAGED_DECODE_NOALLOC_MAX_BYTES];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of the current device's `scratch`, resolved once per device.
int static_scratch(const char* name, void** ptr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return set_error(static_cast<int>(e), "%s: hipGetDevice failed: %s", name,
                     hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return set_error(FK_ERR_UNSUPPORTED, "%s: device %d beyond the %d supported", name, dev,
                     kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess)
      return set_error(static_cast<int>(e), "%s: hipGetSymbolAddress(scratch) failed: %s",
                       name, hipGetErrorString(e));
    if (p == nullptr)
      return set_error(FK_ERR_UNSUPPORTED, "%s: hipGetSymbolAddress(scratch) returned NULL",
                       name);
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return FK_OK;
}

}  // namespace
}  // namespace fk

extern "C" int fk_paged_decode_noalloc(void* out, int64_t out_row_stride, const void* q,
                                       int64_t q_row_stride, const void* k_cache,
                                       const void* v_cache, int kv_dtype, const float* k_scale,
                                       const float* v_scale, const int32_t* block_tables,
                                       int64_t bt_row_stride, const int32_t* ctx_lens,
                                       int64_t batch, int num_heads, int num_kv_heads,
                                       int head_size, int block_size, int64_t num_blocks,
                                       float scale, int window_left, const float* sinks,
                                       int64_t part_tokens, int64_t max_parts, void* stream) {
  const char* name = "fk_paged_decode_noalloc";
  void* ws = nullptr;
  int rc = fk::static_scratch(name, &ws);
  if (rc != FK_OK) return rc;
  rc = fk_paged_decode(out, out_row_stride, q, q_row_stride, k_cache, v_cache, kv_dtype, k_scale,
                       v_scale, block_tables, bt_row_stride, ctx_lens, batch, num_heads,
                       num_kv_heads, head_size, block_size, num_blocks, scale, window_left, sinks,
                       part_tokens, max_parts, ws, FK_PAGED_DECODE_NOALLOC_MAX_BYTES, stream);
  if (rc == FK_ERR_WORKSPACE) {  // the launch needs more than the static scratch holds
    char why[256];
    snprintf(why, sizeof(why), "%s", fk_last_error());
    return fk::set_error(FK_ERR_WORKSPACE,
                         "%s: the launch needs more than the %lld-byte static scratch (%s); "
                         "use fk_paged_decode with a caller-owned workspace",
                         name, (long long)FK_PAGED_DECODE_NOALLOC_MAX_BYTES, why);
  }
  return rc;
}
