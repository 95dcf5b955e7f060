// tl_noalloc.hip -- tl_paged_attention_decode_noalloc: the paged-attention
// decode with its split-K workspace in a library-owned device array, for
// callers that cannot allocate device memory (code under HIP graph capture,
// serving loops, harnesses that forbid hipMalloc).
//
// `scratch` is a file-scope device array of TL_NOALLOC_SCRATCH_BYTES; each
// GPU the library runs on holds its own copy until the process ends.  In
// host code the array's name is only a host-side stand-in, so its device
// address is looked up once per device with hipGetSymbolAddress (with that
// device current) and only that address is handed to the kernels.
//
// The split-K partials need no clearing: the decode writes the (max, sum,
// output) of every partition that a sequence has, and the log-sum-exp merge
// reads only those, so a call never sees an earlier call's contents.  Calls
// that overlap on one GPU (two streams, two threads) share the array and
// race.
#include "tl_attn.h"
#include "tl_internal.hpp"

#include <hip/hip_runtime.h>

#include <mutex>
#include <stdio.h>

namespace {

static __device__ __align__(256) unsigned char scratch[TL_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch[kMaxDevices];   // device address of `scratch`, per device

// The device address of `scratch` on the current device (nullptr on error;
// *err gets the HIP error).
void* scratch_ptr(hipError_t* err) {
  int dev = -1;
  *err = hipGetDevice(&dev);
  if (*err != hipSuccess) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    *err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (*err != hipSuccess) return nullptr;
    g_scratch[dev] = p;
  }
  return g_scratch[dev];
}

thread_local char g_msg[256];

}  // namespace

extern "C" {

int tl_paged_attention_decode_noalloc(const tl_decode_desc* desc, void* out, const void* q,
                                      const void* k_cache, const void* v_cache,
                                      const int32_t* block_tables, const int32_t* seq_lens,
                                      int32_t max_context_len, void* stream) {
  // Argument errors are reported by the decode itself (a NULL workspace of
  // 0 bytes is what it accepts for a single-pass call).
  const size_t need = tl_paged_attention_workspace_bytes(desc, max_context_len);
  if (need == 0)
    return tl_paged_attention_decode(desc, out, q, k_cache, v_cache, block_tables, seq_lens,
                                     max_context_len, nullptr, 0, stream);
  if (need > (size_t)TL_NOALLOC_SCRATCH_BYTES) {
    snprintf(g_msg, sizeof g_msg,
             "split-K workspace of %zu bytes exceeds the %u-byte library scratch "
             "(use tl_paged_attention_decode with a caller workspace)",
             need, (unsigned)TL_NOALLOC_SCRATCH_BYTES);
    return tl::report_error(TL_ERR_INVALID_ARGUMENT, g_msg);
  }
  hipError_t err;
  void* ws = scratch_ptr(&err);
  if (!ws) {
    snprintf(g_msg, sizeof g_msg, "hipGetSymbolAddress of the library scratch failed: %s",
             hipGetErrorString(err));
    return tl::report_error(TL_ERR_BACKEND, g_msg);
  }
  return tl_paged_attention_decode(desc, out, q, k_cache, v_cache, block_tables, seq_lens,
                                   max_context_len, ws, (size_t)TL_NOALLOC_SCRATCH_BYTES, stream);
}

}  // extern "C"
