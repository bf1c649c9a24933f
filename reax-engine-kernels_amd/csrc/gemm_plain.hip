// libreax_plain.so (-DREAX_LIB_PLAIN) and libreax_slices.so (-DREAX_LIB_SLICES) for MI355X: the plain and split-K
// ("slices") bf16 GEMMs behind their config-index C ABIs (libreax_plain/gemm_plain2.cu:31-57,
// libreax_slices/gemm_slices_v2.cu:55-84), on the shared matrix-core tiles (gemm_tile.h: fp32 accumulation in
// ascending K, each output rounded once to its storage type).
//
//   plain:  D[m][n] = X[m][:] . W[n][:]                  X [M][K], W [N][K] row-major, D row stride ldd
//   slices: P[s][m][n] = X[m][s kps, (s+1) kps) . W[n][s kps, (s+1) kps)   P[s] row-major [M][N] at p + s M N,
//           bf16 or fp32 (part_fp32)
//
// The reference selects one of 15 / 16 CUTLASS sm80 tile configurations by index, all with the same results; here
// index 0 runs the tile that is fastest on large products (256 x 256, or 256 x 160 where that fills the CUs better)
// and index c > 0 the gfx950 tile (gemm_tile.h) nearest to the threadblock shape of the reference's config c. All
// tiles give the same bits too, so a caller that times every index and keeps the fastest still chooses among real
// alternatives. An unknown index returns 9, as in the reference.
// Shapes follow CUTLASS's can_implement for 8-wide bf16 accesses (code 1): positive sizes, K (kps) and the output
// row stride multiples of 8; missing buffers and rows not 16-byte aligned also return 1 (the reference faults on
// them). A failed launch returns 4, like the reference's trailing launch-error check.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#pragma GCC visibility push(default)
#if defined(REAX_LIB_PLAIN)
#include "libreax_plain.h"
#elif defined(REAX_LIB_SLICES)
#include "libreax_slices.h"
#else
#error "build with -DREAX_LIB_PLAIN or -DREAX_LIB_SLICES"
#endif
#pragma GCC visibility pop

#include "gemm_tile.h"

namespace reax {
namespace {

__device__ __forceinline__ void put(float* o, float v) { *o = v; }
__device__ __forceinline__ void put(uint16_t* o, float v) { *o = (uint16_t)(pack_bf16x2(v, 0.f) & 0xffffu); }

// grid (tiles_m * tiles_n, 1, S); slice s covers k in [s kext, (s + 1) kext) and writes out + s obs
template <class T, typename OutT>
__global__ void __launch_bounds__(T::THREADS) gemm_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                          OutT* __restrict__ out, int M, int N, int K, int kext,
                                                          long long ldo, long long obs, int tiles_m, int tiles_n) {
  __shared__ __align__(16) typename T::Lds S;
  const int s = blockIdx.z;
  int tm, tn;
  gemm::tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m_blk = tm * T::BM, n_blk = tn * T::BN;
  typename T::Acc acc;
  T::mainloop(S, x, w, K, s * kext, (s + 1) * kext, M, N, m_blk, n_blk, acc);

  // One output per lane per store: accumulating C^T instead (four adjacent outputs per lane, one 8- or 16-byte store
  // each) measured 2-3% slower on every tile.
  const int lane = threadIdx.x & 63, wm = T::wm(), wn = T::wn();
  OutT* o = out + s * obs;
#pragma unroll
  for (int a = 0; a < T::WTM; ++a)
#pragma unroll
    for (int b = 0; b < T::WTN; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m_blk + wm + 32 * a + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        const int col = n_blk + wn + 32 * b + (lane & 31);
        if (row < M && col < N) put(o + row * ldo + col, acc[a][b][v]);
      }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <class T, typename OutT>
int launch_tile(const void* x, const void* w, void* out, int M, int N, int K, int kext, int S, long long ldo,
                long long obs, void* stream) {
  const int tiles_m = (M + T::BM - 1) / T::BM, tiles_n = (N + T::BN - 1) / T::BN;
  if ((long long)tiles_m * tiles_n > INT32_MAX) return 4;  // more tiles than one grid dimension holds
  hipLaunchKernelGGL((gemm_kernel<T, OutT>), dim3((unsigned)(tiles_m * tiles_n), 1, (unsigned)S), dim3(T::THREADS), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w),
                     static_cast<OutT*>(out), M, N, K, kext, ldo, obs, tiles_m, tiles_n);
  return hipGetLastError() == hipSuccess ? 0 : 4;
}

// Compute units of the device that owns the stream (cached per device; 0 if it cannot be queried).
int stream_cus(void* stream) {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (stream ? hipStreamGetDevice(static_cast<hipStream_t>(stream), &dev) != hipSuccess : hipGetDevice(&dev) != hipSuccess)
    return 0;
  if (dev < 0 || dev >= 64) return 0;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 0;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// Config index 0 (the 256 x 256 tile) takes the 256 x 160 tile instead when that takes less time by rounds of the
// grid over the CUs times tile area over per-CU rate. The narrower tile reads more LDS fragments per MFMA (6 per 5
// against 3 per 4) and measured 0.72 of the wide tile's rate per CU; it wins where the wide tile leaves CUs idle
// (N = 2560, M = 4096: 160 tiles of 256 x 256 on 256 CUs against 256 of 256 x 160). All tiles give the same bits.
int pick_wide(int M, int N, int S, void* stream) {
  const int cus = stream_cus(stream);
  if (cus <= 0) return gemm::kD256x256;
  auto rounds = [&](int bm, int bn) {
    return (((long long)(M + bm - 1) / bm) * ((N + bn - 1) / bn) * S + cus - 1) / cus;
  };
  const double t256 = (double)rounds(256, 256) * 256 * 256, t160 = (double)rounds(256, 160) * 256 * 160 / 0.72;
  return t160 < t256 ? gemm::kD256x160 : gemm::kD256x256;
}

template <typename OutT>
int launch(int tile, const void* x, const void* w, void* out, int M, int N, int K, int kext, int S, long long ldo,
           long long obs, void* stream) {
  if (kext % gemm::BK) tile = gemm::kT128x128;  // the ring tiles copy whole 64-deep slices only
  else if (tile == gemm::kD256x256) tile = pick_wide(M, N, S, stream);
  switch (tile) {
    case gemm::kD128x128: return launch_tile<gemm::D128x128, OutT>(x, w, out, M, N, K, kext, S, ldo, obs, stream);
    case gemm::kD256x128: return launch_tile<gemm::D256x128, OutT>(x, w, out, M, N, K, kext, S, ldo, obs, stream);
    case gemm::kD128x256: return launch_tile<gemm::D128x256, OutT>(x, w, out, M, N, K, kext, S, ldo, obs, stream);
    case gemm::kD256x256: return launch_tile<gemm::D256x256, OutT>(x, w, out, M, N, K, kext, S, ldo, obs, stream);
    case gemm::kD256x160: return launch_tile<gemm::D256x160, OutT>(x, w, out, M, N, K, kext, S, ldo, obs, stream);
    default: return launch_tile<gemm::T128x128, OutT>(x, w, out, M, N, K, kext, S, ldo, obs, stream);
  }
}

}  // namespace
}  // namespace reax

namespace reax {
namespace {
constexpr const char* kWideName = "mfma 256x256x64 (256x160x64 where that fills the CUs better), 8 waves, LDS ring";
}  // namespace
}  // namespace reax

extern "C" {

#if defined(REAX_LIB_PLAIN)
// tile of each config: 0 the 256 x 256 ring tile; the others by the reference's threadblock shapes
// (gemm_plain2.cu:40-54) 256x128, 128x128, 128x256, 128x256, 192x128, 192x128, 64x256, 64x256, 128x128, 128x128
// (warp 64x32), 256x128, 256x64, 128x64, 64x128
static const unsigned char kPlainTile[15] = {4, 2, 1, 3, 3, 2, 2, 3, 3, 1, 0, 2, 2, 1, 0};

int reax_gemm_ncfg(void) { return 15; }
const char* reax_gemm_cfgname(int c) {
  return c == 0 ? reax::kWideName : (c > 0 && c < 15) ? reax::gemm::kTileNames[kPlainTile[c]] : "?";
}

int reax_gemm(int cfg, const void* x, const void* w, void* d, int M, int N, int K, int ldd, void* stream) {
  if (cfg < 0 || cfg >= 15) return 9;  // gemm_plain2.cu:56
  if (M <= 0 || N <= 0 || K <= 0 || K % 8 || ldd % 8 || ldd < N || !x || !w || !d || !reax::aligned16(x) ||
      !reax::aligned16(w) || (reinterpret_cast<uintptr_t>(d) & 1u))
    return 1;  // can_implement (gemm_plain2.cu:24)
  return reax::launch<uint16_t>(kPlainTile[cfg], x, w, d, M, N, K, K, 1, ldd, 0, stream);
}

#else
// tile of each config: 0 the 256 x 256 ring tile; the others by the reference's threadblock shapes
// (gemm_slices_v2.cu:38-53) 256x128, 128x128, 64x256, 128x128, 256x128, 128x256, 64x128, 128x64, 64x256, 64x128,
// 256x64, 128x128, 128x128, 64x128, 256x128
static const unsigned char kSlicesTile[16] = {4, 2, 1, 3, 1, 2, 3, 0, 1, 3, 0, 2, 1, 1, 0, 2};

int reax_slices_ncfg(void) { return 16; }
const char* reax_slices_cfgname(int c) {
  return c == 0 ? reax::kWideName : (c > 0 && c < 16) ? reax::gemm::kTileNames[kSlicesTile[c]] : "?";
}

int reax_slices(int cfg, int part_fp32, const void* x, const void* w, void* p, int M, int N, int kps, int S, int K,
                void* stream) {
  if (cfg < 0 || cfg >= 16) return 9;  // gemm_slices_v2.cu:83
  if (M <= 0 || N <= 0 || kps <= 0 || S <= 0 || S > 65535 || kps % 8 || N % 8 || K % 8 || (long long)kps * S > K ||
      !x || !w || !p || !reax::aligned16(x) || !reax::aligned16(w) ||
      (reinterpret_cast<uintptr_t>(p) & (part_fp32 ? 3u : 1u)))
    return 1;  // can_implement (gemm_slices_v2.cu:29)
  const long long obs = (long long)M * N;
  return part_fp32 ? reax::launch<float>(kSlicesTile[cfg], x, w, p, M, N, K, kps, S, N, obs, stream)
                   : reax::launch<uint16_t>(kSlicesTile[cfg], x, w, p, M, N, K, kps, S, N, obs, stream);
}
#endif

}  // extern "C"
