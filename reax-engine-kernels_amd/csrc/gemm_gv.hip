// libreax_gv.so for MI355X: the Qwen3.5 MLP gate/up GEMM with its SiLU-times-up epilogue fused. Replaces reax_gv,
// libreax_gv/gateup_vis2.cu:172-209.
//
//   C = X W^T   (X [M][K] row-major; W [2*N2][K] row-major with gate and up rows interleaved in groups of 4:
//                rows 8j..8j+3 gate features 4j..4j+3, rows 8j+4..8j+7 the matching up features, gv:1-6)
//   out[m][4j + i] = bf16(bf16(silu(bf16(C[m][8j + i]))) * bf16(C[m][8j + 4 + i])),  silu(g) = g / (1 + exp(-g))
// with fp32 accumulation on the matrix cores (the reference: CUTLASS sm80 with ascending K; the orders differ, so
// agreement is to fp32 accumulation accuracy) and SiLU defined as bf16(g / fp32(1 + exp(-g))) evaluated exactly to
// that definition (an fp32 fast path with a double-precision fallback at bf16 rounding boundaries; the reference's
// expf is accurate to about an ulp, so its bf16 SiLU can differ by one ulp in rare elements).
//
// Kernel: the shared matrix-core tiles (gemm_tile.h: 128 x 128 up to 256 x 256 tiles of C, K in slices of 64 copied
// straight into an LDS ring, the config index picks the tile) with an epilogue that
// pairs each gate column with the up column four to its right (four lanes over in the accumulator layout) and writes
// only the activations: no intermediate buffer, like the reference's visitor.
#include <hip/hip_runtime.h>
#include <stdint.h>

#pragma GCC visibility push(default)
#include "libreax_gv.h"
#pragma GCC visibility pop

#include "gemm_tile.h"

namespace reax {
namespace {

__device__ __forceinline__ float bfr(float x) { return bf16lo(pack_bf16x2(x, 0.f)); }

// bf16(g / fp32(1 + exp(-g))) for a bf16 g (same construction as the conv kernel's SiLU: exact 16-bit split of
// log2 e against the 8-bit g, v_exp_f32 with a second-order correction, v_rcp_f32; within 9 ulp of the defined
// fp32 quotient, and the double-precision definition decides within 32 ulp of a bf16 midpoint)
__device__ __attribute__((noinline)) float silu_bf16_slow(float y) {
  const float d = (float)(1.0 + exp(-(double)y));
  return bfr(y / d);
}
__device__ __forceinline__ float silu_bf16(float y) {
  if (!(y > -64.0f && y < 64.0f)) return silu_bf16_slow(y);
  const float a_hi = y * -1.44268798828125f;
  const float a_lo = y * -7.052607543300837e-06f;
  const float t = a_lo * 0.6931471824645996f;
  const float eh = fast_exp2(a_hi);
  const float e = __builtin_fmaf(eh, __builtin_fmaf(0.5f * t, t, t), eh);
  const float q = y * __builtin_amdgcn_rcpf(1.0f + e);
  const uint32_t low = __float_as_uint(q) & 0xffffu;
  if (low > 0x8000u - 32u && low < 0x8000u + 32u) return silu_bf16_slow(y);
  return bfr(q);
}

template <class T>
__global__ void __launch_bounds__(T::THREADS) gv_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                        uint16_t* __restrict__ out, int M, int N2, int K, int tiles_m,
                                                        int tiles_n) {
  __shared__ __align__(16) typename T::Lds S;
  const int NC = 2 * N2;  // columns of C
  int tm, tn;
  gemm::tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m_blk = tm * T::BM, n_blk = tn * T::BN;
  typename T::Acc acc;
  T::mainloop(S, x, w, K, 0, K, M, NC, m_blk, n_blk, acc);
  const int lane = threadIdx.x & 63, wm = T::wm(), wn = T::wn();

  // ---- epilogue: element v of tile (a, b) is C[row][col] with row = wm + 32a + 8(v/4) + 4(lane/32) + v%4 and
  // col = wn + 32b + lane%32; gate columns have col % 8 < 4 and their up column is col + 4 (lane + 4)
  const int j = lane & 31;
#pragma unroll
  for (int a = 0; a < T::WTM; ++a)
#pragma unroll
    for (int b = 0; b < T::WTN; ++b)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float up = __shfl(acc[a][b][v], lane + 4 < 64 ? lane + 4 : lane, 64);
        const int row = m_blk + wm + 32 * a + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        const int col = n_blk + wn + 32 * b + j;
        if ((col & 7) < 4 && row < M && col < NC) {
          const float gb = bfr(acc[a][b][v]), ub = bfr(up);
          const float act = bfr(silu_bf16(gb) * ub);
          out[(long long)row * N2 + (col >> 3) * 4 + (col & 3)] = (uint16_t)(pack_bf16x2(act, 0.f) & 0xffffu);
        }
      }
}

template <class T>
int launch_tile(const void* x, const void* w, void* out, int M, int N2, int K, void* stream) {
  const int tiles_m = (M + T::BM - 1) / T::BM, tiles_n = (int)((2LL * N2 + T::BN - 1) / T::BN);
  if ((long long)tiles_m * tiles_n > INT32_MAX) return 3;  // more tiles than one grid dimension holds
  hipLaunchKernelGGL(gv_kernel<T>, dim3((unsigned)(tiles_m * tiles_n)), dim3(T::THREADS), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w),
                     static_cast<uint16_t*>(out), M, N2, K, tiles_m, tiles_n);
  return hipGetLastError() == hipSuccess ? 0 : 3;  // gv:167
}

}  // namespace
}  // namespace reax

extern "C" {

// tile of each config: 0 the 256 x 256 ring tile; the others by the reference's threadblock shapes (gv:186-205)
// 256x128, 128x128, 128x256, 128x256, 256x128, 128x128, 128x128, 64x256, 128x256, 128x192, 128x192, 192x128, 192x128,
// 64x256, 64x256, 192x192, 128x128, 128x128 (warp 64x32), 256x128
static const unsigned char kGvTile[20] = {4, 2, 1, 3, 3, 2, 1, 1, 3, 3, 3, 3, 2, 2, 3, 3, 4, 1, 0, 2};

int reax_gv_ncfg(void) { return 20; }
const char* reax_gv_cfgname(int c) { return (c >= 0 && c < 20) ? reax::gemm::kTileNames[kGvTile[c]] : "?"; }

int reax_gv(int cfg, const void* x, const void* w, void* out, int M, int N2, int K, void* stream) {
  if (cfg < 0 || cfg >= 20) return 9;  // gv:207
  if (K % 8 || N2 % 4) return 1;       // gv:143
  // empty or negative sizes, 2 N2 beyond int, missing or misaligned buffers (16-byte row loads): the reference's
  // kernel cannot take them either (an empty grid fails to launch, its int problem size overflows, misaligned loads
  // fault)
  if (M <= 0 || N2 <= 0 || N2 > INT32_MAX / 2 || K <= 0 || !x || !w || !out || (reinterpret_cast<uintptr_t>(x) & 15u) ||
      (reinterpret_cast<uintptr_t>(w) & 15u) || (reinterpret_cast<uintptr_t>(out) & 1u))
    return 3;
  using namespace reax::gemm;
  const int tile = K % BK ? kT128x128 : kGvTile[cfg];  // the ring tiles copy whole 64-deep slices only
  switch (tile) {
    case kD128x128: return reax::launch_tile<D128x128>(x, w, out, M, N2, K, stream);
    case kD256x128: return reax::launch_tile<D256x128>(x, w, out, M, N2, K, stream);
    case kD128x256: return reax::launch_tile<D128x256>(x, w, out, M, N2, K, stream);
    case kD256x256: return reax::launch_tile<D256x256>(x, w, out, M, N2, K, stream);
    default: return reax::launch_tile<T128x128>(x, w, out, M, N2, K, stream);
  }
}

}  // extern "C"
