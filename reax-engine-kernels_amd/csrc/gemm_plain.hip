// libreax_plain.so (-DREAX_LIB_PLAIN) and libreax_slices.so (-DREAX_LIB_SLICES) for MI355X: the plain and split-K
// ("slices") bf16 GEMMs behind their config-index C ABIs (libreax_plain/gemm_plain2.cu:31-57,
// libreax_slices/gemm_slices_v2.cu:55-84), on the shared matrix-core tile (gemm_tile.h: fp32 accumulation in
// ascending K, each output rounded once to its storage type).
//
//   plain:  D[m][n] = X[m][:] . W[n][:]                  X [M][K], W [N][K] row-major, D row stride ldd
//   slices: P[s][m][n] = X[m][s kps, (s+1) kps) . W[n][s kps, (s+1) kps)   P[s] row-major [M][N] at p + s M N,
//           bf16 or fp32 (part_fp32)
//
// The reference selects one of 15 / 16 CUTLASS sm80 tile configurations by index, all with the same results; the
// index is validated the same way here (an unknown index returns 9) and every index runs the one gfx950 tile.
// Shapes follow CUTLASS's can_implement for 8-wide bf16 accesses (code 1): positive sizes, K (kps) and the output
// row stride multiples of 8; missing buffers and rows not 16-byte aligned also return 1 (the reference faults on
// them). A failed launch returns 4, like the reference's trailing launch-error check.
#include <hip/hip_runtime.h>
#include <stdint.h>

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

// grid (ceil(N / 128), ceil(M / 128), S); slice s covers k in [s kext, (s + 1) kext) and writes out + s obs
template <typename OutT>
__global__ void __launch_bounds__(gemm::THREADS) gemm_kernel(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ w, OutT* __restrict__ out,
                                                             int M, int N, int K, int kext, long long ldo,
                                                             long long obs) {
  __shared__ __align__(16) gemm::Lds S;
  const int s = blockIdx.z;
  const int m_blk = blockIdx.y * gemm::BM, n_blk = blockIdx.x * gemm::BN;
  f32x16_t acc[2][2];
  gemm::mainloop(S, x, w, K, s * kext, (s + 1) * kext, M, N, m_blk, n_blk, acc);

  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int wm = 64 * (wv >> 1), wn = 64 * (wv & 1);
  OutT* o = out + s * obs;
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = m_blk + wm + 32 * a + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        const int col = n_blk + wn + 32 * b + (lane & 31);
        if (row < M && col < N) put(o + row * ldo + col, acc[a][b][v]);
      }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <typename OutT>
int launch(const void* x, const void* w, void* out, int M, int N, int K, int kext, int S, long long ldo,
           long long obs, void* stream) {
  const dim3 grid((unsigned)((N + gemm::BN - 1) / gemm::BN), (unsigned)((M + gemm::BM - 1) / gemm::BM), (unsigned)S);
  hipLaunchKernelGGL(gemm_kernel<OutT>, grid, dim3(gemm::THREADS), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), static_cast<OutT*>(out), M, N,
                     K, kext, ldo, obs);
  return hipGetLastError() == hipSuccess ? 0 : 4;
}

}  // namespace
}  // namespace reax

extern "C" {

#if defined(REAX_LIB_PLAIN)
int reax_gemm_ncfg(void) { return 15; }
const char* reax_gemm_cfgname(int c) {
  static const char* n[] = {"mfma 128x128x64 cfg0",  "mfma 128x128x64 cfg1",  "mfma 128x128x64 cfg2",
                            "mfma 128x128x64 cfg3",  "mfma 128x128x64 cfg4",  "mfma 128x128x64 cfg5",
                            "mfma 128x128x64 cfg6",  "mfma 128x128x64 cfg7",  "mfma 128x128x64 cfg8",
                            "mfma 128x128x64 cfg9",  "mfma 128x128x64 cfg10", "mfma 128x128x64 cfg11",
                            "mfma 128x128x64 cfg12", "mfma 128x128x64 cfg13", "mfma 128x128x64 cfg14"};
  return (c >= 0 && c < 15) ? n[c] : "?";
}

int reax_gemm(int cfg, const void* x, const void* w, void* d, int M, int N, int K, int ldd, void* stream) {
  if (cfg < 0 || cfg >= 15) return 9;  // gemm_plain2.cu:56
  if (M <= 0 || N <= 0 || K <= 0 || K % 8 || ldd % 8 || ldd < N || !x || !w || !d || !reax::aligned16(x) ||
      !reax::aligned16(w) || (reinterpret_cast<uintptr_t>(d) & 1u))
    return 1;  // can_implement (gemm_plain2.cu:24)
  return reax::launch<uint16_t>(x, w, d, M, N, K, K, 1, ldd, 0, stream);
}

#else
int reax_slices_ncfg(void) { return 16; }
const char* reax_slices_cfgname(int c) {
  static const char* n[] = {"mfma 128x128x64 cfg0",  "mfma 128x128x64 cfg1",  "mfma 128x128x64 cfg2",
                            "mfma 128x128x64 cfg3",  "mfma 128x128x64 cfg4",  "mfma 128x128x64 cfg5",
                            "mfma 128x128x64 cfg6",  "mfma 128x128x64 cfg7",  "mfma 128x128x64 cfg8",
                            "mfma 128x128x64 cfg9",  "mfma 128x128x64 cfg10", "mfma 128x128x64 cfg11",
                            "mfma 128x128x64 cfg12", "mfma 128x128x64 cfg13", "mfma 128x128x64 cfg14",
                            "mfma 128x128x64 cfg15"};
  return (c >= 0 && c < 16) ? n[c] : "?";
}

int reax_slices(int cfg, int part_fp32, const void* x, const void* w, void* p, int M, int N, int kps, int S, int K,
                void* stream) {
  if (cfg < 0 || cfg >= 16) return 9;  // gemm_slices_v2.cu:83
  if (M <= 0 || N <= 0 || kps <= 0 || S <= 0 || S > 65535 || kps % 8 || N % 8 || K % 8 || (long long)kps * S > K ||
      !x || !w || !p || !reax::aligned16(x) || !reax::aligned16(w) ||
      (reinterpret_cast<uintptr_t>(p) & (part_fp32 ? 3u : 1u)))
    return 1;  // can_implement (gemm_slices_v2.cu:29)
  const long long obs = (long long)M * N;
  return part_fp32 ? reax::launch<float>(x, w, p, M, N, K, kps, S, N, obs, stream)
                   : reax::launch<uint16_t>(x, w, p, M, N, K, kps, S, N, obs, stream);
}
#endif

}  // extern "C"
