// The matrix-core tiles shared by the GEMM libraries (libreax_plain.so, libreax_slices.so, libreax_gv.so):
//   C[m][n] = sum_{k0 <= k < k1} X[m][k] W[n][k]   for one BM x BN tile of C
// with X [.][ldx] and W [.][ldx] row-major bf16 (both operands K-contiguous), fp32 accumulation.
//
// A tile is NWM x NWN wavefronts, each a (32 WTM) x (32 WTN) block of C as WTM x WTN v_mfma_f32_32x32x16_bf16
// tiles, so that one 16-deep step reads WTM + WTN fragments for WTM * WTN MFMAs (larger wave blocks need less LDS
// bandwidth per MFMA). K advances 64 at a time: the BM x 64 and BN x 64 slices of X and W live in LDS (16-byte units
// XOR-swizzled by row, so every MFMA fragment is one conflict-free 16-byte read), one barrier per slice. Tile stages
// a slice through registers (read while the previous slice is multiplied; rows beyond M or N and k units at or
// beyond k1 read as zeros; k0 and k1 multiples of 8); DmaTile copies slices straight into an LDS ring (below).
//
// Every tile shape adds each accumulator's K slices in the same ascending order of 16-element MFMA steps, so all
// shapes give identical bits; against another summation order results agree to fp32 accumulation accuracy.
//
// Accumulator layout: element v of acc[a][b] is C[wm + 32a + 8(v/4) + 4(lane/32) + v%4][wn + 32b + lane%32]
// relative to the tile, with wm = 32 WTM (wave / NWN), wn = 32 WTN (wave % NWN).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fmha_common.h"
#include "fmha_tiles.h"

#include <type_traits>

namespace reax {
namespace gemm {

constexpr int BK = 64;
constexpr int UNITS = BK / 8;  // 16-byte units per slice row

// element offset of (row r, unit u) in a slice of rows of 64: units XOR row % 8, so 8 consecutive rows read by one
// fragment use 8 distinct 16-byte columns
__device__ __forceinline__ int slot(int r, int u) { return r * BK + ((u ^ (r & (UNITS - 1))) << 3); }

template <int NWM_, int NWN_, int WTM_, int WTN_>
struct Tile {
  static constexpr int NWM = NWM_, NWN = NWN_, WTM = WTM_, WTN = WTN_;
  static constexpr int THREADS = 64 * NWM * NWN;
  static constexpr int BM = 32 * WTM * NWM, BN = 32 * WTN * NWN;
  static constexpr int LX = BM * UNITS / THREADS, LW = BN * UNITS / THREADS;  // staged units per thread
  static_assert(BM * UNITS % THREADS == 0 && BN * UNITS % THREADS == 0, "whole units per thread");

  struct Lds {
    uint16_t xs[2][BM * BK];
    uint16_t ws[2][BN * BK];
  };
  using Acc = f32x16_t[WTM][WTN];

  __device__ static int wm() { return 32 * WTM * ((int)(threadIdx.x >> 6) / NWN); }
  __device__ static int wn() { return 32 * WTN * ((int)(threadIdx.x >> 6) % NWN); }

  __device__ __forceinline__ static void mainloop(Lds& S, const uint16_t* __restrict__ x,
                                                  const uint16_t* __restrict__ w, long long ldx, int k0, int k1,
                                                  int M, int N, int m_blk, int n_blk, Acc& acc) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wm0 = wm(), wn0 = wn();
    struct Regs {
      u32x4_t x[LX], w[LW];
    };
    auto load = [&](Regs& R, int kb) __attribute__((always_inline)) {
#pragma unroll
      for (int e = 0; e < LX; ++e) {
        const int i = tid + THREADS * e, r = i / UNITS, k = kb + 8 * (i % UNITS), gm = m_blk + r;
        R.x[e] = (gm < M && k < k1) ? *reinterpret_cast<const u32x4_t*>(x + gm * ldx + k) : u32x4_t{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int e = 0; e < LW; ++e) {
        const int i = tid + THREADS * e, r = i / UNITS, k = kb + 8 * (i % UNITS), gn = n_blk + r;
        R.w[e] = (gn < N && k < k1) ? *reinterpret_cast<const u32x4_t*>(w + gn * ldx + k) : u32x4_t{0u, 0u, 0u, 0u};
      }
    };
    auto store = [&](const Regs& R, int buf) __attribute__((always_inline)) {
#pragma unroll
      for (int e = 0; e < LX; ++e) {
        const int i = tid + THREADS * e;
        *reinterpret_cast<u32x4_t*>(&S.xs[buf][slot(i / UNITS, i % UNITS)]) = R.x[e];
      }
#pragma unroll
      for (int e = 0; e < LW; ++e) {
        const int i = tid + THREADS * e;
        *reinterpret_cast<u32x4_t*>(&S.ws[buf][slot(i / UNITS, i % UNITS)]) = R.w[e];
      }
    };
    auto compute = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks) {
        const int u = 2 * ks + (lane >> 5), r = lane & 31;
        bf16x8_t af[WTM], bf[WTN];
#pragma unroll
        for (int a = 0; a < WTM; ++a)
          af[a] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(&S.xs[buf][slot(wm0 + 32 * a + r, u)]));
#pragma unroll
        for (int b = 0; b < WTN; ++b)
          bf[b] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(&S.ws[buf][slot(wn0 + 32 * b + r, u)]));
#pragma unroll
        for (int a = 0; a < WTM; ++a)
#pragma unroll
          for (int b = 0; b < WTN; ++b) acc[a][b] = mfma32(af[a], bf[b], acc[a][b]);
      }
    };

#pragma unroll
    for (int a = 0; a < WTM; ++a)
#pragma unroll
      for (int b = 0; b < WTN; ++b)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;

    // slice kt + 1 is read into registers while slice kt (LDS buffer kt % 2) is multiplied. Reading two slices
    // ahead (a second register set) measured slower on every shape: the loads arrive in time already.
    const int nk = (k1 - k0 + BK - 1) / BK;
    Regs R;
    load(R, k0);
    store(R, 0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      if (kt + 1 < nk) load(R, k0 + (kt + 1) * BK);
      compute(kt & 1);
      if (kt + 1 < nk) {
        store(R, (kt + 1) & 1);  // buffer (kt + 1) % 2 was last read in step kt - 1, before its closing barrier
        __syncthreads();
      }
    }
  }
};

// The same tile with the K slices copied straight from global memory into LDS (global_load_lds_dwordx4, no
// register staging) through a ring of NS slices, NS - 1 slices ahead of the multiply. The copy of a 1 KB chunk
// (8 rows of a 64-wide slice) puts lane l's 16 bytes at chunk + 16 l, so lane l fetches the unit that the XOR
// swizzle places there: row 8 c + l / 8, unit (l % 8) ^ (row % 8). The copies are issued as inline assembly, which
// the compiler does not track: each wavefront waits for its own copies with s_waitcnt vmcnt (they complete in issue
// order) and the barrier that follows makes every wavefront's copies visible. Rows beyond M or N read the last
// valid row (their outputs are never stored); the K extent must be a whole number of slices (no zero fill).
template <int NWM_, int NWN_, int WTM_, int WTN_, int NS_>
struct DmaTile {
  static constexpr int NWM = NWM_, NWN = NWN_, WTM = WTM_, WTN = WTN_, NS = NS_;
  static constexpr int THREADS = 64 * NWM * NWN, NWAVES = NWM * NWN;
  static constexpr int BM = 32 * WTM * NWM, BN = 32 * WTN * NWN;
  static constexpr int XCH = BM / 8, CH = (BM + BN) / 8;  // 1 KB chunks of X, of the whole slice
  static constexpr int CPW = (CH + NWAVES - 1) / NWAVES;   // chunks copied per wavefront per slice (at most)
  static constexpr bool EVEN = CPW * NWAVES == CH;         // otherwise the last wavefronts copy one fewer
  static_assert(NS == 2 || NS == 3, "two or three slices in the ring");
  static constexpr int CLAST = CH - (NWAVES - 1) * CPW;  // chunks of the last wavefront (CPW when EVEN)
  static_assert(CLAST > 0 && CLAST <= CPW, "every wavefront copies at least one chunk");

  struct Lds {
    uint16_t xs[NS][BM * BK];
    uint16_t ws[NS][BN * BK];
  };
  using Acc = f32x16_t[WTM][WTN];

  __device__ static int wm() { return 32 * WTM * ((int)(threadIdx.x >> 6) / NWN); }
  __device__ static int wn() { return 32 * WTN * ((int)(threadIdx.x >> 6) % NWN); }

  __device__ __forceinline__ static void mainloop_pinned(Lds& S, const uint16_t* __restrict__ x,
                                                  const uint16_t* __restrict__ w, long long ldx, int k0, int k1,
                                                  int M, int N, int m_blk, int n_blk, Acc& acc) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm0 = wm(), wn0 = wn();
    // copy i (of this wavefront's CPW) of slice kb into ring slot st: chunk wv * CPW + i
    auto copy_one = [&](int st, int kb, int i) __attribute__((always_inline)) {
      const int c = wv * CPW + i;
      if (!EVEN && c >= CH) return;  // wavefront-uniform
      const bool isx = c < XCH;
      const int r = 8 * (isx ? c : c - XCH) + (lane >> 3);
      const int u = (lane & 7) ^ (r & 7);
      const int row = isx ? min(m_blk + r, M - 1) : min(n_blk + r, N - 1);
      const uint16_t* src = (isx ? x : w) + (long long)row * ldx + kb + 8 * u;
      const uint32_t m0 = __builtin_amdgcn_readfirstlane(
          (uint32_t)reinterpret_cast<uintptr_t>(isx ? &S.xs[st][c * 512] : &S.ws[st][(c - XCH) * 512]));
      asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(m0) : "memory");
    };
    // The slice multiply in a fixed issue order: one slot per MFMA (NM = 4 WTM WTN per slice, 16-deep step major,
    // then a, b), scheduling barriers between slots. Step ks + 1's fragments are read during step ks (read q of
    // R = WTM + WTN in slot q G / R of the step's G = WTM WTN slots, W's first), and the copies of a later slice go out one
    // every NM / CPW slots: neither the reads nor the copies come in a burst that holds the matrix core up.
    constexpr int G = WTM * WTN, R = WTM + WTN, NKS = BK / 16, NM = NKS * G;
    auto compute = [&](int st, auto&& cp) __attribute__((always_inline)) {
      const int r = lane & 31, hsel = lane >> 5;
      bf16x8_t fr[2][R];
      auto read = [&](auto ksc, auto qc) __attribute__((always_inline)) {
        constexpr int ks = decltype(ksc)::value, q = decltype(qc)::value;
        const int u = 2 * ks + hsel;
        if constexpr (q < WTM)
          fr[ks & 1][q] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(&S.xs[st][slot(wm0 + 32 * q + r, u)]));
        else
          fr[ks & 1][q] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(&S.ws[st][slot(wn0 + 32 * (q - WTM) + r, u)]));
      };
      static_for<0, R>([&](auto qc) __attribute__((always_inline)) { read(std::integral_constant<int, 0>{}, qc); });
      __builtin_amdgcn_sched_barrier(0);
      static_for<0, NM>([&](auto ic) __attribute__((always_inline)) {
        constexpr int i = decltype(ic)::value;
        constexpr int ks = i / G, j = i % G, a = j / WTN, b = j % WTN;
        acc[a][b] = mfma32(fr[ks & 1][a], fr[ks & 1][WTM + b], acc[a][b]);
        if constexpr (ks + 1 < NKS) {
          // the W fragments first: every MFMA of a step uses one of them, the X fragments come in order of use
          static_for<0, R>([&](auto pc) __attribute__((always_inline)) {
            constexpr int pq = decltype(pc)::value;
            constexpr int q = pq < WTN ? WTM + pq : pq - WTN;
            if constexpr (pq * G / R == j) read(std::integral_constant<int, ks + 1>{}, std::integral_constant<int, q>{});
          });
        }
        static_for<0, CPW>([&](auto cc) __attribute__((always_inline)) {
          constexpr int c = decltype(cc)::value;
          if constexpr ((c * NM) / CPW == i) cp(c);
        });
        __builtin_amdgcn_sched_barrier(0);
      });
    };
#pragma unroll
    for (int a = 0; a < WTM; ++a)
#pragma unroll
      for (int b = 0; b < WTN; ++b)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;

    const int nk = (k1 - k0) / BK;
    // prologue: slices 0 .. NS - 2 in flight; wait for slice 0
#pragma unroll
    for (int j = 0; j < NS - 1; ++j)
      if (j < nk)
#pragma unroll
        for (int i = 0; i < CPW; ++i) copy_one(j, k0 + j * BK, i);
    if (NS == 2 || nk == 1)
      __builtin_amdgcn_s_waitcnt(vmcnt_le(0));
    else if (EVEN || wv < NWAVES - 1)
      __builtin_amdgcn_s_waitcnt(vmcnt_le(CPW));  // slice 1's copies may still be in flight
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_le(CLAST));
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      // slot (kt + NS - 1) % NS was last read in step kt - 1, before its closing barrier
      const bool more = kt + NS - 1 < nk;
      const int stn = (kt + NS - 1) % NS, kbn = k0 + (kt + NS - 1) * BK;
      compute(kt % NS, [&](int i) __attribute__((always_inline)) {
        if (more) copy_one(stn, kbn, i);
      });
      if (kt + 1 < nk) {
        // slice kt + 1 must have landed; slice kt + 2 (NS = 3, if there is one: this wavefront's copies of it) may
        // still be in flight
        if (NS == 3 && kt + 2 < nk) {
          if (EVEN || wv < NWAVES - 1)
            __builtin_amdgcn_s_waitcnt(vmcnt_le(CPW));
          else
            __builtin_amdgcn_s_waitcnt(vmcnt_le(CLAST));
        } else {
          __builtin_amdgcn_s_waitcnt(vmcnt_le(0));
        }
        __syncthreads();
      }
    }
  }

  __device__ __forceinline__ static void mainloop(Lds& S, const uint16_t* __restrict__ x,
                                                  const uint16_t* __restrict__ w, long long ldx, int k0, int k1,
                                                  int M, int N, int m_blk, int n_blk, Acc& acc) {
    // tiles with 5 or more MFMAs per 16-deep step take the fixed issue order; those with 4 (two 32-row by two
    // 32-column blocks per wavefront) measured faster with the compiler's own order and all copies at the start
    if constexpr (WTM * WTN >= 5) {
      mainloop_pinned(S, x, w, ldx, k0, k1, M, N, m_blk, n_blk, acc);
      return;
    }
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm0 = wm(), wn0 = wn();
    // copy slice kb into ring slot st: chunks wv * CPW .. wv * CPW + CPW - 1
    auto copy = [&](int st, int kb) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < CPW; ++i) {
        const int c = wv * CPW + i;
        if (!EVEN && c >= CH) break;  // wavefront-uniform
        const bool isx = c < XCH;
        const int r = 8 * (isx ? c : c - XCH) + (lane >> 3);
        const int u = (lane & 7) ^ (r & 7);
        const int row = isx ? min(m_blk + r, M - 1) : min(n_blk + r, N - 1);
        const uint16_t* src = (isx ? x : w) + (long long)row * ldx + kb + 8 * u;
        const uint32_t m0 = __builtin_amdgcn_readfirstlane(
            (uint32_t)reinterpret_cast<uintptr_t>(isx ? &S.xs[st][c * 512] : &S.ws[st][(c - XCH) * 512]));
        asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(m0) : "memory");
      }
    };
    auto compute = [&](int st) __attribute__((always_inline)) {
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks) {
        const int u = 2 * ks + (lane >> 5), r = lane & 31;
        bf16x8_t af[WTM], bf[WTN];
#pragma unroll
        for (int a = 0; a < WTM; ++a)
          af[a] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(&S.xs[st][slot(wm0 + 32 * a + r, u)]));
#pragma unroll
        for (int b = 0; b < WTN; ++b)
          bf[b] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(&S.ws[st][slot(wn0 + 32 * b + r, u)]));
#pragma unroll
        for (int a = 0; a < WTM; ++a)
#pragma unroll
          for (int b = 0; b < WTN; ++b) acc[a][b] = mfma32(af[a], bf[b], acc[a][b]);
      }
    };
#pragma unroll
    for (int a = 0; a < WTM; ++a)
#pragma unroll
      for (int b = 0; b < WTN; ++b)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;

    const int nk = (k1 - k0) / BK;
    // prologue: slices 0 .. NS - 2 in flight; wait for slice 0
#pragma unroll
    for (int j = 0; j < NS - 1; ++j)
      if (j < nk) copy(j, k0 + j * BK);
    if (NS == 2 || nk == 1)
      __builtin_amdgcn_s_waitcnt(vmcnt_le(0));
    else if (EVEN || wv < NWAVES - 1)
      __builtin_amdgcn_s_waitcnt(vmcnt_le(CPW));  // slice 1's copies may still be in flight
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_le(CLAST));
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      // slot (kt + NS - 1) % NS was last read in step kt - 1, before its closing barrier
      if (kt + NS - 1 < nk) copy((kt + NS - 1) % NS, k0 + (kt + NS - 1) * BK);
      compute(kt % NS);
      if (kt + 1 < nk) {
        // slice kt + 1 must have landed; slice kt + 2 (NS = 3, if there is one: this wavefront's copies of it) may
        // still be in flight
        if (NS == 3 && kt + 2 < nk) {
          if (EVEN || wv < NWAVES - 1)
            __builtin_amdgcn_s_waitcnt(vmcnt_le(CPW));
          else
            __builtin_amdgcn_s_waitcnt(vmcnt_le(CLAST));
        } else {
          __builtin_amdgcn_s_waitcnt(vmcnt_le(0));
        }
        __syncthreads();
      }
    }
  }
};

// The tiles a config index can select (measured at the MLP shapes of the GEMM bench leg: the 8-wavefront 256 x 256
// ring tile is the fastest there; 3-slice rings, which fit one workgroup per CU, and 4-wavefront 256 x 256 tiles,
// which spill, were slower). Register staging remains for K extents that are not whole slices.
using T128x128 = Tile<2, 2, 2, 2>;            // 4 wavefronts, register-staged, 64 KB LDS (two workgroups per CU)
using D128x128 = DmaTile<2, 2, 2, 2, 2>;      // 4 wavefronts, 64 KB
using D256x128 = DmaTile<4, 2, 2, 2, 2>;      // 8 wavefronts of 64 x 64, 96 KB
using D128x256 = DmaTile<2, 4, 2, 2, 2>;      // 8 wavefronts of 64 x 64, 96 KB
using D256x256 = DmaTile<2, 4, 4, 2, 2>;      // 8 wavefronts of 128 x 64, 128 KB
using D256x160 = DmaTile<8, 1, 1, 5, 3>;      // 8 wavefronts of 32 x 160, 3 slices, 156 KB (fills 256 CUs at N = 2560)
enum TileId : unsigned char { kT128x128 = 0, kD128x128 = 1, kD256x128 = 2, kD128x256 = 3, kD256x256 = 4, kD256x160 = 5 };
constexpr const char* kTileNames[6] = {"mfma 128x128x64, 4 waves, register-staged", "mfma 128x128x64, 4 waves, LDS ring",
                                       "mfma 256x128x64, 8 waves, LDS ring", "mfma 128x256x64, 8 waves, LDS ring",
                                       "mfma 256x256x64, 8 waves, LDS ring", "mfma 256x160x64, 8 waves, LDS ring"};

// XCD-aware tile order: hardware hands consecutive workgroups to the 8 XCDs in turn, so workgroup b runs on XCD
// b % 8. When the tile count is a multiple of 8, each XCD is given a contiguous range of the tile sequence; the
// sequence walks columns of GROUP_M tile rows, so the workgroups resident on one XCD share X rows and W rows in that
// XCD's L2. A bijection of [0, tiles_m * tiles_n) onto the tile grid.
__device__ __forceinline__ void tile_of(int b, int tiles_m, int tiles_n, int& tm, int& tn) {
  constexpr int XCDS = 8, GROUP_M = 8;
  const int nb = tiles_m * tiles_n;
  const int t = nb % XCDS == 0 ? (b % XCDS) * (nb / XCDS) + b / XCDS : b;
  const int per_group = GROUP_M * tiles_n;
  const int first_m = (t / per_group) * GROUP_M, rows = min(tiles_m - first_m, GROUP_M), i = t % per_group;
  tm = first_m + i % rows;
  tn = i / rows;
}

}  // namespace gemm
}  // namespace reax
