// Split-KV behind the drop-in entry points at short query blocks (reax_fmha_q / reax_fmha_qp with at most 32 folded
// rows per (batch, KV head): the engine's decode step is Lq 1 x G 8 = 8 rows).
//
// The reference launches one CTA per (KV head, batch, 64-row block) (reax_fmha_v8.cu:428, reax_fmha_v11.cu:559), so
// a decode step streams each (b, KV head)'s whole key range through one CU: with config 5's model (2 KV heads) at
// batch 1 that is 2 CUs of 256 pulling 67 MB (1.8 ms measured, 37.6 GB/s). Here the key range is cut into splits
// that fill the GPU (fmha_decode_kernel, P wavefronts per split merged in LDS), and an LSE-weighted combine kernel
// merges the splits and applies the output store of the entry point (folded O, or reax_fmha_qp's gate epilogue).
//
// The split partials need device memory the drop-in ABI has no argument for, and the reference allocates nothing.
// They go to `short_scratch`, a file-scope device array (SHORT_SLOTS slots of SHORT_SLOT_BYTES; each GPU the
// library runs on holds its own copy until the process ends). Calls on one GPU share it, so every use of a slot is
// ordered on the GPU after its previous use: each call's stream waits on the slot's event before the split kernel
// and records it again after the combine kernel. A call takes the slot last used by a stream with its handle (the
// wait is then within one stream), else a slot whose last use has finished, else the least recently used slot
// (its stream then queues behind that use). Nothing is allocated on the call path after a slot's event has been
// created (once per slot and device); a stream under graph capture, a short key range or a shape whose partials
// exceed a slot runs the unsplit kernel instead.
#include <hip/hip_runtime.h>

#include <climits>
#include <mutex>

#include "fmha_launch.h"

namespace reax {

constexpr int SHORT_SLOTS = 4;
constexpr size_t SHORT_SLOT_BYTES = size_t(8) << 20;
constexpr int SHORT_BN = 32;          // keys per tile of the head_dim-256 decode kernel
constexpr int SHORT_MIN_TILES = 2;    // key tiles per wavefront at least
constexpr int SHORT_WAVES_PER_CU = 4; // the decode kernel's 4 wavefronts, one workgroup per CU (128 KB of LDS)

static __device__ __align__(256) uint8_t short_scratch[SHORT_SLOTS * SHORT_SLOT_BYTES];

namespace {

struct DeviceSlots {
  std::mutex mu;
  uint8_t* base = nullptr;  // device address of short_scratch on this device, once looked up
  bool lookup_failed = false;
  unsigned long long owner[SHORT_SLOTS] = {};  // handle of the stream of slot i's last use
  hipEvent_t done[SHORT_SLOTS] = {};          // recorded on that stream after slot i's last use
  unsigned long long last[SHORT_SLOTS] = {};
  unsigned long long tick = 0;
};
DeviceSlots g_slots[64];

// Split shape for the decode kernel: about SHORT_WAVES_PER_CU wavefronts per CU in all, each over at least
// SHORT_MIN_TILES key tiles; P = 1, 2 or 4 wavefronts per split; split_len a multiple of P tiles; no empty split;
// the partials within one slot. False when fewer than two wavefronts per (b, KV head) would result.
bool short_shape(const FwdParams& p, int cus, int& P, int& splits, int& split_len) {
  const long long nt = ((long long)p.N + SHORT_BN - 1) / SHORT_BN;
  const long long bh = (long long)p.B * p.H;
  if (nt <= 0 || bh <= 0) return false;
  long long want = ((long long)SHORT_WAVES_PER_CU * cus + bh - 1) / bh;  // wavefronts per (b, KV head)
  want = std::min(want, std::max(1ll, nt / SHORT_MIN_TILES));
  if (want < 2) return false;
  P = want >= 4 ? 4 : want >= 2 ? 2 : 1;
  long long sp = (want + P - 1) / P;
  const long long per_split = bh * p.M * (long long)(256 + 1) * 4 + 512;  // partial O + LSE (+ alignment)
  const long long fit = (long long)SHORT_SLOT_BYTES / per_split;
  if (fit < 1) return false;
  sp = std::min(sp, fit);
  const long long tpw = (nt + sp * P - 1) / (sp * P);  // tiles per wavefront
  const long long len = tpw * P * SHORT_BN;
  if (len > INT_MAX) return false;
  sp = ((long long)p.N + len - 1) / len;
  if (sp * P < 2) return false;
  splits = (int)sp;
  split_len = (int)len;
  return splitkv_workspace_bytes(p.B, p.H, p.M, 256, splits) <= SHORT_SLOT_BYTES;
}

// Device address of short_scratch on device `dev` (with that device current; the array's name is only a host-side
// stand-in). Called with d.mu held.
uint8_t* scratch_base(DeviceSlots& d, int dev) {
  if (d.base || d.lookup_failed) return d.base;
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess) return nullptr;
  if (cur != dev && hipSetDevice(dev) != hipSuccess) return nullptr;
  void* q = nullptr;
  const hipError_t rc = hipGetSymbolAddress(&q, HIP_SYMBOL(short_scratch));
  if (cur != dev) (void)hipSetDevice(cur);
  if (rc != hipSuccess || !q) {
    d.lookup_failed = true;
    return nullptr;
  }
  d.base = static_cast<uint8_t*>(q);
  return d.base;
}

}  // namespace

int launch_short_split(const FwdParams& p0, bool post, hipStream_t stream) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return SHORT_NOT_TAKEN;
  const int cus = device_cus(stream);
  if (cus <= 0) return SHORT_NOT_TAKEN;
  int P = 1, splits = 1, split_len = SHORT_BN;
  if (!short_shape(p0, cus, P, splits, split_len)) return SHORT_NOT_TAKEN;
  int dev = -1;
  if ((stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev)) != hipSuccess || dev < 0 || dev >= 64)
    return SHORT_NOT_TAKEN;
  const unsigned long long sid = (unsigned long long)reinterpret_cast<uintptr_t>(stream);
  DeviceSlots& d = g_slots[dev];
  std::lock_guard<std::mutex> lock(d.mu);
  uint8_t* base = scratch_base(d, dev);
  if (!base) return SHORT_NOT_TAKEN;
  // a slot last used on this stream, else one whose last use has finished, else the least recently used one
  int slot = -1;
  for (int i = 0; i < SHORT_SLOTS && slot < 0; ++i)
    if (d.done[i] && d.owner[i] == sid) slot = i;
  for (int i = 0; i < SHORT_SLOTS && slot < 0; ++i)
    if (!d.done[i] || hipEventQuery(d.done[i]) == hipSuccess) slot = i;
  if (slot < 0) {
    slot = 0;
    for (int i = 1; i < SHORT_SLOTS; ++i)
      if (d.last[i] < d.last[slot]) slot = i;
  }
  if (!d.done[slot] && hipEventCreateWithFlags(&d.done[slot], hipEventDisableTiming) != hipSuccess) {
    d.done[slot] = nullptr;
    return SHORT_NOT_TAKEN;
  }
  // always wait, also when the slot's last use was on a stream with this handle: a handle can name a new stream
  // after the old one was destroyed with work pending, and the wait costs nothing measurable (the ~6 us between a
  // preceding kernel and the split kernel in a kernel trace is there with or without it)
  if (const int rc = (int)hipStreamWaitEvent(stream, d.done[slot], 0)) return rc;
  FwdParams p = p0;
  p.num_splits = splits;
  p.split_len = split_len;
  set_workspace(p, base + (size_t)slot * SHORT_SLOT_BYTES, 256);
  if (const int rc = launch_decode_split(p, 256, P, post, stream)) return rc;
  if (const int rc = (int)hipEventRecord(d.done[slot], stream)) return rc;
  d.owner[slot] = sid;
  d.last[slot] = ++d.tick;
  return 0;
}

}  // namespace reax
