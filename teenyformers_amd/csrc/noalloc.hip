// The causal flash-attention backward for callers that cannot allocate
// device memory (code under HIP graph capture, serving loops, harnesses that
// forbid hipMalloc): the workspace teeny_causal_flash_attn2_bwd takes from
// its caller is a fixed device array of this library instead.
//
// This file is compiled by hipcc as host code plus a device part that holds
// only `scratch`; the HIP runtime gives each device its own copy of the array
// when it loads this file's code object, and hipGetSymbolAddress returns that
// device's address.  That address, never the host-side name `scratch`, is
// what reaches kernels; teeny_init asks for it on each device, and the entry
// point refuses a device where that has not happened
// (TEENY_ERR_NOT_INITIALIZED) rather than loading anything itself.  Every
// call on a device shares its array: calls that overlap on one device (two
// streams, two threads) race on it.  Nothing in
// the array has to start at zero: the dQ kernel writes every LSE / Delta slot
// (padding included) before the dK/dV kernel reads it, and split partial sums
// are written whole before the merge reads them.
#include <hip/hip_runtime.h>

#include <mutex>

#include "teeny_hip.h"

// capi.cpp: records a failed HIP call for teeny_last_hip_error; whether the
// current device's code objects are loaded (teeny_init has run on it)
extern "C" __attribute__((visibility("hidden"))) void teeny_set_last_hip_error(int e);
extern "C" __attribute__((visibility("hidden"))) int teeny_device_ready(void);

namespace {

constexpr size_t kScratchBytes = (size_t)16 << 20;  // 16 MiB per device
constexpr int kMaxDevices = 64;

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// The current device's address of `scratch`, asked once per device with that
// device current, from teeny_init.
extern "C" __attribute__((visibility("hidden"))) int teeny_scratch_setup(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    teeny_set_last_hip_error((int)e);
    return TEENY_ERR_HIP;
  }
  if (dev < 0 || dev >= kMaxDevices) return TEENY_ERR_HIP;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      teeny_set_last_hip_error((int)e);
      (void)hipGetLastError();
      return TEENY_ERR_HIP;
    }
    g_scratch_ptr[dev] = p;
  }
  if (out) *out = g_scratch_ptr[dev];
  return TEENY_OK;
}

extern "C" {

size_t teeny_scratch_bytes(void) { return kScratchBytes; }

int teeny_causal_flash_attn2_bwd_noalloc(const void* q, const void* k, const void* v,
                                         const void* o, const void* dout, const float* l,
                                         void* dq, void* dk, void* dv, int n_ctx_q, int n_ctx_k,
                                         float softmax_scale, int batch, int n_heads_q,
                                         int n_heads_kv, int head_dim, int dtype,
                                         hipStream_t stream) {
  const size_t need =
      teeny_flash_attn2_bwd_workspace_bytes(n_ctx_q, batch, n_heads_q, head_dim, dtype);
  if (need > kScratchBytes) return TEENY_ERR_SCRATCH;
  // set up by teeny_init on this device, or refused: loading code objects or
  // asking for the array's address here would allocate and synchronise,
  // which is what this entry point's callers (graph capture) cannot have
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    teeny_set_last_hip_error((int)e);
    return TEENY_ERR_HIP;
  }
  if (dev < 0 || dev >= kMaxDevices) return TEENY_ERR_HIP;
  void* ws = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    ws = g_scratch_ptr[dev];
  }
  if (!ws || !teeny_device_ready()) return TEENY_ERR_NOT_INITIALIZED;
  // the whole array: a GQA split that fits in it is used, as the allocating
  // entry point does with a workspace of this size
  return teeny_causal_flash_attn2_bwd(q, k, v, o, dout, l, dq, dk, dv, n_ctx_q, n_ctx_k,
                                      softmax_scale, batch, n_heads_q, n_heads_kv, head_dim,
                                      dtype, ws, kScratchBytes, stream);
}

}  // extern "C"
