// noalloc.hip — moe_layer_forward for callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc): the layer's workspace is a static device array instead
// of a caller buffer.
//
// The array, `scratch`, is kScratchBytes of file-scope device memory that
// every GPU the library runs on holds until the process ends. Its device
// address is looked up once per device, with that device current, on the
// entry point's first call there (hipGetSymbolAddress), and only that address
// is ever handed to kernels or copies: in host code the array's name is a
// host-side stand-in, not a device address.
//
// Every call on a GPU shares that GPU's array, which keeps the last call's
// contents. The layer's kernels write every workspace byte they read, so
// nothing needs clearing between calls. Calls that overlap on one GPU (on
// different streams, or from several host threads) race on the array and
// must be serialised by the caller.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <mutex>

#include "../../include/moe_hip.h"
#include "moe_internal.hpp"

namespace moe {
moe_status layer_forward_in_order(const moe_layer_desc* d, const void* x, int32_t T, void* y,
                                  void* ws, size_t ws_bytes, const moe_layer_trace* tr,
                                  hipStream_t st);
size_t layer_workspace_bytes(const moe_layer_desc* d, int32_t T);
}  // namespace moe

// 16 MiB: a Qwen3-MoE-shaped layer (hidden 2048, 128 experts, top-8,
// intermediate 768) needs 14 MB at 256 tokens, a GPT-OSS-20B-shaped one
// 3.7 MB at 64 tokens.
static constexpr size_t kScratchBytes = 16u << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch[kMaxDevices];  // device address of `scratch` per device, once looked up

moe_status failf(moe_status s, const char* fmt, ...) {
  char buf[320];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  moe::set_error_text(buf);
  return s;
}

// The current device's address of `scratch` (looked up on its first use).
moe_status scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return failf(MOE_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return failf(MOE_ERR_UNSUPPORTED, "moe_layer_forward_noalloc: device %d beyond %d", dev,
                 kMaxDevices);
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return failf(MOE_ERR_HIP, "moe_layer_forward_noalloc: scratch address lookup: %s",
                   hipGetErrorString(e));
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return MOE_OK;
}

}  // namespace

extern "C" size_t moe_layer_noalloc_max_bytes(void) { return kScratchBytes; }

extern "C" moe_status moe_layer_forward_noalloc(const moe_layer_desc* d, const void* x, int32_t T,
                                                void* y, const moe_layer_trace* trace,
                                                hipStream_t stream) {
  if (T <= 0)
    return failf(MOE_ERR_INVALID, "MoELayer.decodeMany: T must be positive (got %d)", T);
  const size_t need = moe::layer_workspace_bytes(d, T);
  if (need == 0) return moe_validate_layer(d);  // sets the reason
  if (need > kScratchBytes)
    return failf(MOE_ERR_WORKSPACE,
                 "moe_layer_forward_noalloc: the layer needs %zu bytes of workspace at T=%d, "
                 "above the static scratch of %zu bytes; use moe_layer_forward",
                 need, T, kScratchBytes);
  void* ws = nullptr;
  const moe_status s = scratch_address(&ws);
  if (s != MOE_OK) return s;
  return moe::layer_forward_in_order(d, x, T, y, ws, kScratchBytes, trace, stream);
}
