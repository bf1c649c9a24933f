// Internal host-side launch interface shared by the C-ABI entry points.
#pragma once
#include <hip/hip_runtime.h>

#include "fmha_common.h"

#include <initializer_list>

namespace reax {

// Launches the forward kernel for head_dim 128 or 256 in one of the mask modes (MaskMode). Asynchronous on
// `stream`; returns 0 or a hipError_t code (hipErrorInvalidValue for unsupported shapes or misaligned rows,
// hipErrorInvalidConfiguration for an empty grid, as the reference's zero-sized launch would report).
int launch_fwd(const FwdParams& p, int head_dim, int mode, bool post, hipStream_t stream);

// The head_dim-256 wavefront-pair kernel (qpos or varlen mode, optional POST epilogue) on an already prepared
// FwdParams (fmha_fwd_pair.hip).
int launch_fwd_pair(const FwdParams& p, int mode, bool post, hipStream_t stream);

// Compute units of the device that owns `stream`, 0 if it cannot be queried (the persistent kernels launch one
// workgroup per CU).
int device_cus(hipStream_t stream);

// True when `ptr` and every stride are multiples of n_elems_multiple bf16 elements.
static inline bool aligned_elems(const void* ptr, long long n_elems_multiple, std::initializer_list<long long> strides) {
  if ((reinterpret_cast<uintptr_t>(ptr) & (uintptr_t)(2 * n_elems_multiple - 1)) != 0) return false;
  for (long long s : strides)
    if (s % n_elems_multiple != 0) return false;
  return true;
}

// Split-KV forward for short query blocks (decode): partial results per key split go to `ws`, then an LSE
// combine kernel writes O (bf16) and the optional LSE (fmha_fwd.hip).
struct SplitParams {
  FwdParams f;     // q/k/v/o/lse, qpos, strides, B, H, G, M, N (rows per (b, kv head) = M)
  int num_splits;  // key splits per (b, kv head)
  void* ws;        // workspace (see splitkv_workspace_bytes)
  size_t ws_bytes;
};
size_t splitkv_workspace_bytes(int B, int H, int M, int head_dim, int num_splits);
int launch_splitkv(const SplitParams& p, int head_dim, hipStream_t stream);

// The same with the library's per-device static scratch as the workspace (p.ws / p.ws_bytes are ignored): no
// allocation anywhere on the call path. Returns hipErrorOutOfMemory when the workspace the shape needs exceeds
// SPLITKV_SCRATCH_BYTES (fmha_noalloc.hip).
constexpr size_t SPLITKV_SCRATCH_BYTES = size_t(8) << 20;
int launch_splitkv_noalloc(SplitParams p, int head_dim, hipStream_t stream);

}  // namespace reax
