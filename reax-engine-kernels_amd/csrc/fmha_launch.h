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

// The decode kernel + combine kernel on a prepared FwdParams whose num_splits, split_len (a multiple of P key tiles:
// 64 keys at head_dim 128, 32 at 256), ws_o and ws_lse are set; P = 1, 2 or 4 wavefronts per split, p.M <= 32.
// post: the combine applies reax_fmha_qp's gate epilogue (head_dim 256) instead of storing O / LSE.
int launch_decode_split(FwdParams p, int head_dim, int P, bool post, hipStream_t stream);
// Points p.ws_o / p.ws_lse into a workspace laid out as splitkv_workspace_bytes describes (p.num_splits set).
void set_workspace(FwdParams& p, void* ws, int head_dim);

// The drop-in entry points at short query blocks (head_dim 256, qpos mode, at most 32 folded rows per (b, KV
// head), e.g. one decode token of 8 query heads): split-KV through the library's static per-device scratch, with
// the split count chosen to fill the GPU (fmha_short.hip). Returns SHORT_NOT_TAKEN when the call should run
// unsplit instead (short key ranges, a stream being captured, the scratch in use by another stream's unfinished
// call, a shape whose partials exceed a scratch slot), else 0 or a hipError_t code.
constexpr int SHORT_NOT_TAKEN = -1000;
int launch_short_split(const FwdParams& p, bool post, hipStream_t stream);

// The same with the library's per-device static scratch as the workspace (p.ws / p.ws_bytes are ignored): no
// allocation anywhere on the call path. Returns hipErrorOutOfMemory when the workspace the shape needs exceeds
// SPLITKV_SCRATCH_BYTES (fmha_noalloc.hip).
constexpr size_t SPLITKV_SCRATCH_BYTES = size_t(8) << 20;
int launch_splitkv_noalloc(SplitParams p, int head_dim, hipStream_t stream);

}  // namespace reax
