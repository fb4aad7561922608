// mla_decode_fwd_noalloc: the whole decode (Q quant, plan, decode, combine)
// with its workspace in a file-scope device array instead of a caller buffer,
// for callers that cannot allocate device memory (code under HIP graph
// capture, serving loops, harnesses that forbid hipMalloc).  No reference
// counterpart.
//
// The array lives in this library's code object: each device the library
// runs on holds its own copy (kNoAllocScratchBytes) from the first use until
// the process ends.  Host code never passes the array's name to a kernel (on
// the host it is only a stand-in for the symbol); its device address is
// looked up once per device with hipGetSymbolAddress, with that device
// current, and only that address is used.  Nothing in the pipeline needs the
// scratch to start zeroed (every word a kernel reads was written earlier in the
// same call), so no clearing is done.  Calls on one device share the array:
// calls that overlap on a device (different streams, or different threads
// without ordering) race.
#include <mutex>

#include "../../include/mla_mi355x.h"
#include "mla_internal.hpp"

namespace mla {
namespace {

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {nullptr};
std::mutex g_scratch_mutex;

// device address of this device's scratch (looked up on first use per device)
int scratch_ptr(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(MLA_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return set_error(MLA_ERR_UNSUPPORTED, "device ordinal %d too large", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return set_error(MLA_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    if (p == nullptr || (reinterpret_cast<uintptr_t>(p) & 255u) != 0)
      return set_error(MLA_ERR_HIP, "scratch symbol address %p is not 256-byte aligned", p);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MLA_OK;
}

}  // namespace
}  // namespace mla

using namespace mla;

extern "C" {

int64_t mla_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

int mla_decode_fwd_noalloc(const void* q_bf16, const void* k_cache, int64_t k_row_stride, const void* k_scales,
                           int64_t k_scale_stride, const void* v_cache, int64_t v_row_stride,
                           const float* kv_scale, const int32_t* kv_indptr, const int32_t* kv_indices, int batch,
                           int q_seq_len, int num_heads, float sm_scale, int kv_mode, void* out_bf16,
                           float* lse_out, void* stream) {
  int64_t need = 0;
  int rc = mla_workspace_bytes(batch, num_heads, kv_mode, &need);
  if (rc) return rc;
  if (need > kNoAllocScratchBytes)
    return set_error(MLA_ERR_WORKSPACE_TOO_SMALL,
                     "this shape needs a %lld-byte workspace; mla_decode_fwd_noalloc holds %lld bytes "
                     "(use mla_decode_fwd with a caller workspace)",
                     (long long)need, (long long)kNoAllocScratchBytes);
  void* ws = nullptr;
  if ((rc = scratch_ptr(&ws))) return rc;
  return mla_decode_fwd(q_bf16, k_cache, k_row_stride, k_scales, k_scale_stride, v_cache, v_row_stride, kv_scale,
                        kv_indptr, kv_indices, batch, q_seq_len, num_heads, sm_scale, kv_mode, ws,
                        kNoAllocScratchBytes, out_bf16, lse_out, stream);
}

}  // extern "C"
