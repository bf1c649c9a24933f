// The matrix-core tile shared by the GEMM libraries (libreax_plain.so, libreax_slices.so, libreax_gv.so):
//   C[m][n] = sum_{k0 <= k < k1} X[m][k] W[n][k]   for one 128 x 128 tile of C
// with X [.][ldx] and W [.][ldx] row-major bf16 (both operands K-contiguous), fp32 accumulation.
//
// 256 threads (4 wavefronts), each wavefront a 64 x 64 quarter of the tile as 2 x 2 v_mfma_f32_32x32x16_bf16
// tiles. K advances 64 at a time: the 128 x 64 slices of X and W live in LDS (16-byte units XOR-swizzled by row,
// so every MFMA fragment is one conflict-free 16-byte read), double-buffered, and the next slice is read from
// global memory into registers while the current one is multiplied (one barrier per slice). Rows beyond M or N and
// k units at or beyond k1 read as zeros; k0 and k1 are multiples of 8 (whole 16-byte units).
//
// Each accumulator adds its K slices in ascending order (the MFMA sums 16 products per step), so results agree with
// any fp32-accumulated product to fp32 accumulation accuracy; they are not bit-identical to another order.
//
// Accumulator layout: element v of acc[a][b] is C[wm + 32a + 8(v/4) + 4(lane/32) + v%4][wn + 32b + lane%32]
// relative to the tile, with wm = 64 (wave / 2), wn = 64 (wave % 2).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fmha_common.h"

namespace reax {
namespace gemm {

constexpr int BM = 128, BN = 128, BK = 64, THREADS = 256;
constexpr int UNITS = BK / 8;                       // 16-byte units per slice row
constexpr int LOADS = BM * UNITS / THREADS;         // units per thread per operand per slice (4)
static_assert(BM == BN && BM * UNITS % THREADS == 0, "one staging pattern serves both operands");

struct Lds {
  uint16_t xs[2][BM * BK];
  uint16_t ws[2][BN * BK];
};

// element offset of (row r, unit u) in a 128 x 64 slice
__device__ __forceinline__ int slot(int r, int u) { return r * BK + ((u ^ (r & (UNITS - 1))) << 3); }

__device__ __forceinline__ void mainloop(Lds& S, const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                         long long ldx, int k0, int k1, int M, int N, int m_blk, int n_blk,
                                         f32x16_t (&acc)[2][2]) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = 64 * (wv >> 1), wn = 64 * (wv & 1);
  u32x4_t rx[LOADS], rw[LOADS];
  auto load = [&](int kb) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < LOADS; ++e) {
      const int i = tid + THREADS * e, r = i / UNITS, u = i % UNITS, k = kb + 8 * u;
      const int gm = m_blk + r, gn = n_blk + r;
      rx[e] = (gm < M && k < k1) ? *reinterpret_cast<const u32x4_t*>(x + gm * ldx + k) : u32x4_t{0u, 0u, 0u, 0u};
      rw[e] = (gn < N && k < k1) ? *reinterpret_cast<const u32x4_t*>(w + gn * ldx + k) : u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  auto store = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < LOADS; ++e) {
      const int i = tid + THREADS * e, r = i / UNITS, u = i % UNITS;
      *reinterpret_cast<u32x4_t*>(&S.xs[buf][slot(r, u)]) = rx[e];
      *reinterpret_cast<u32x4_t*>(&S.ws[buf][slot(r, u)]) = rw[e];
    }
  };

#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;

  const int nk = (k1 - k0 + BK - 1) / BK;
  load(k0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load(k0 + (kt + 1) * BK);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int u = 2 * ks + (lane >> 5), r = lane & 31;
      bf16x8_t af[2], bf[2];
#pragma unroll
      for (int a = 0; a < 2; ++a)
        af[a] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(&S.xs[buf][slot(wm + 32 * a + r, u)]));
#pragma unroll
      for (int b = 0; b < 2; ++b)
        bf[b] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(&S.ws[buf][slot(wn + 32 * b + r, u)]));
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[a][b] = mfma32(af[a], bf[b], acc[a][b]);
    }
    if (kt + 1 < nk) {
      store(buf ^ 1);  // the other buffer was last read in the previous iteration, before its closing barrier
      __syncthreads();
    }
  }
}

}  // namespace gemm
}  // namespace reax
