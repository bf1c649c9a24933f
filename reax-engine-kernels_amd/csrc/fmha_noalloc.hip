// Split-KV decode without a caller workspace: the partial results live in a file-scope device array.
//
// For callers that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc): reax_fmha_splitkv_noalloc runs the same kernels as reax_fmha_splitkv, with `scratch` below as the
// workspace. Each GPU the library runs on holds its own copy of the array (SPLITKV_SCRATCH_BYTES) until the process
// ends. Every call on one GPU shares that GPU's copy, and it keeps the last call's contents: calls that overlap on
// one GPU (different streams without ordering, or several host threads) race on it. The split kernels write every
// partial they later read, so nothing needs clearing between calls.
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

#include "fmha_launch.h"

namespace reax {

static __device__ __align__(256) uint8_t scratch[SPLITKV_SCRATCH_BYTES];

// Device address of `scratch` on device `dev`, looked up once per device with that device current (the array's
// name is only a host-side stand-in: passing it to a kernel would fault). nullptr if the lookup fails.
static void* scratch_address(int dev) {
  static std::atomic<void*> addr[64];
  static std::mutex mu;
  if (dev < 0 || dev >= 64) return nullptr;
  void* p = addr[dev].load(std::memory_order_acquire);
  if (p) return p;
  std::lock_guard<std::mutex> lock(mu);
  p = addr[dev].load(std::memory_order_relaxed);
  if (p) return p;
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess) return nullptr;
  if (cur != dev && hipSetDevice(dev) != hipSuccess) return nullptr;
  void* q = nullptr;
  const hipError_t rc = hipGetSymbolAddress(&q, HIP_SYMBOL(scratch));
  if (cur != dev) (void)hipSetDevice(cur);
  if (rc != hipSuccess || q == nullptr) return nullptr;
  addr[dev].store(q, std::memory_order_release);
  return q;
}

int launch_splitkv_noalloc(SplitParams sp, int head_dim, hipStream_t stream) {
  const size_t need = splitkv_workspace_bytes(sp.f.B, sp.f.H, sp.f.M, head_dim, sp.num_splits);
  if (need == 0) return (int)hipErrorInvalidValue;
  if (need > SPLITKV_SCRATCH_BYTES) return (int)hipErrorOutOfMemory;  // larger than the static scratch
  int dev = -1;
  if ((stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev)) != hipSuccess) return (int)hipErrorInvalidDevice;
  void* ws = scratch_address(dev);
  if (!ws) return (int)hipErrorInvalidDevice;
  sp.ws = ws;
  sp.ws_bytes = SPLITKV_SCRATCH_BYTES;
  return launch_splitkv(sp, head_dim, stream);
}

}  // namespace reax
