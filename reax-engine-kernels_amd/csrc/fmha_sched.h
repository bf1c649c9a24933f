// Item schedule of the persistent forward kernels for packed variable-length batches (cu_seqlens).
//
// An item is one row tile (BM folded rows) of one (sequence, KV head) pair. Causal attention makes an item's cost
// the number of 64-key tiles its last row sees, so items differ by up to the longest sequence's tile count. With
// one workgroup per CU and items taken in a fixed order, a workgroup that draws long items late finishes long
// after the others (8 sequences of 592..1811 tokens: a fixed order left a workgroup 45
// tile-steps of work against an average of 25).
//
// Every workgroup computes the same schedule in its prologue, from cu_seqlens alone (no allocation, no atomics):
//   1. sequences sorted by item count, longest first (ties by index); pairs j = rank * H + head in that order;
//   2. the pairs are dealt to NX = 8 classes in a snake (0..7, 7..0, ...), one class per XCD (workgroups are
//      dealt to the 8 XCDs round-robin, so class x is the workgroups with index = x mod 8): a pair's K/V is then
//      read by one XCD only and stays in its L2 (spread over every XCD, config 3's 19 MB of K/V thrashed the
//      4 MB L2s and ran slower than the fixed order despite the better balance);
//   3. within a class, items in "level" order: level i = the i-th row tile of a pair, highest level first, and
//      within a level the class's pairs that reach it (a prefix of its pair list); costs never increase along this
//      order, up to the last, partial tile of a sequence;
//   4. batched longest-processing-time assignment within the class: round r hands the class's items
//      [r PW, r PW + PW) to its PW workgroups in increasing order of the work they already hold (ties by index).
// On config 3 the busiest workgroup gets 34 tile-steps, against 30.5 for the longest single item.
// Shapes beyond the LDS tables (VS_NSEQ sequences, VS_NPAIR pairs per class, VS_TMAX tiles per sequence,
// VS_PMAX workgroups, VS_RMAX rounds) keep the fixed order.
#pragma once
#include <climits>

#include "fmha_common.h"

namespace reax {

constexpr int VS_NSEQ = 256, VS_NPAIR = 256, VS_TMAX = 1024, VS_PMAX = 256, VS_RMAX = 64;

struct VarlenSched {
  int sorted[VS_NSEQ];     // sequence index by rank (most items first)
  int Ts[VS_NSEQ];         // items of the sequence of each rank
  int Ls[VS_NSEQ];         // tokens of the sequence of each rank
  int pref[VS_NPAIR + 1];  // prefix sums of the class's pair item counts
  int cnt[VS_TMAX];        // the class's pairs with more than i items (they reach level i)
  int start[VS_TMAX];      // first position of level i in the class's item order
  alignas(16) int load[VS_PMAX];  // work held by each workgroup of the class (half tile-steps; INT_MAX past pw)
  int mine[VS_RMAX];       // this workgroup's item position in round r, -1 for none
  int ok, nx, tmax, nreal, rounds, npc;
};

// k-th pair of class x of nx (snake deal): pairs 0..nx-1 go to classes 0..nx-1, pairs nx..2nx-1 to nx-1..0, ...
__device__ __forceinline__ int vs_pair(int k, int x, int nx) {
  return 2 * nx * (k >> 1) + ((k & 1) ? 2 * nx - 1 - x : x);
}

// Item at position k of the class's level order -> (rank of its sequence, KV head, row tile = level).
__device__ __forceinline__ void vs_decode(const VarlenSched& S, int H, int x, int k, int& rank, int& head,
                                          int& level) {
  // start[] decreases as the level rises and level i holds positions [start[i], start[i] + cnt[i]) =
  // [start[i], start[i - 1]): the item's level is the lowest one whose start is <= k
  int lo = 0, hi = S.tmax - 1;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (S.start[mid] <= k) hi = mid; else lo = mid + 1;
  }
  level = lo;
  const int j = vs_pair(k - S.start[lo], x, S.nx);
  rank = j / H;
  head = j - rank * H;
}

// Cost of an item in half tile-steps: its key tiles plus a fixed per-item overhead (prologue, epilogue).
__device__ __forceinline__ int vs_cost(const VarlenSched& S, int BM, int G, int rank, int level) {
  const int last = min((level + 1) * (BM / G), S.Ls[rank]) - 1;
  return 2 * (last / 64 + 1) + 3;
}

// Builds this workgroup's schedule (every thread of the workgroup calls it; it ends with a barrier). Sets S.ok = 0
// when the shape exceeds the tables. wg is the workgroup index, P the grid size.
template <int BM>
__device__ void vs_build(VarlenSched& S, const int* cu, int nseq, int H, int G, int P, int wg) {
  const int tid = threadIdx.x, nt = blockDim.x;
  if (nseq > VS_NSEQ || P > VS_PMAX || nseq <= 0 || H <= 0 || BM % G != 0) {
    if (tid == 0) S.ok = 0;
    __syncthreads();
    return;
  }
  const int nx = (P % 8 == 0) ? 8 : 1, x = wg % nx, pw = P / nx, me = wg / nx;
  // items and tokens per sequence, staged in cnt[] and start[] (VS_TMAX >= VS_NSEQ): cu_seqlens is read once
  for (int s = tid; s < nseq; s += nt) {
    const int L = cu[s + 1] - cu[s];
    S.cnt[s] = L > 0 ? (int)(((long long)L * G + BM - 1) / BM) : 0;
    S.start[s] = L;
  }
  __syncthreads();
  for (int s = tid; s < nseq; s += nt) {
    const int T = S.cnt[s];
    int r = 0;
    for (int u = 0; u < nseq; ++u) {
      const int Tu = S.cnt[u];
      r += (Tu > T || (Tu == T && u < s)) ? 1 : 0;
    }
    S.sorted[r] = s;
    S.Ts[r] = T;
    S.Ls[r] = S.start[s];
  }
  __syncthreads();
  if (tid == 0) {
    // the class's pairs, in deal order (their item counts never increase along it)
    const int npairs = nseq * H;
    int n = 0, acc = 0;
    while (n <= VS_NPAIR) {
      const int j = vs_pair(n, x, nx);
      if (j >= npairs) break;
      if (n < VS_NPAIR) S.pref[n] = acc;
      acc += S.Ts[j / H];
      ++n;
    }
    const bool fits = n <= VS_NPAIR;
    if (fits) S.pref[n] = acc;
    S.nx = nx;
    S.npc = n;
    S.tmax = n > 0 ? S.Ts[vs_pair(0, x, nx) / H] : 0;
    S.nreal = acc;
    S.rounds = (acc + pw - 1) / pw;
    S.ok = (fits && S.tmax <= VS_TMAX && S.rounds <= VS_RMAX) ? 1 : 0;
  }
  __syncthreads();
  if (!S.ok) return;
  const int tmax = S.tmax, npc = S.npc;
  // cnt[i] = the class's pairs with more than i items (a prefix of its pair list)
  for (int i = tid; i < tmax; i += nt) {
    int lo = 0, hi = npc;  // first pair with at most i items
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (S.Ts[vs_pair(mid, x, nx) / H] > i) lo = mid + 1; else hi = mid;
    }
    S.cnt[i] = lo;
  }
  __syncthreads();
  // start[i] = items on levels above i = sum over the pairs reaching level i + 1 of (items - (i + 1))
  for (int i = tid; i < tmax; i += nt) {
    const int c = i + 1 < tmax ? S.cnt[i + 1] : 0;
    S.start[i] = S.pref[c] - c * (i + 1);
  }
  for (int m = tid; m < VS_PMAX; m += nt) S.load[m] = m < pw ? 0 : INT_MAX;
  for (int r = tid; r < VS_RMAX; r += nt) S.mine[r] = -1;
  __syncthreads();
  for (int r = 0; r < S.rounds; ++r) {
    int add = 0, pos = -1;
    const int m = tid;
    if (m < pw) {
      const int lm = S.load[m];
      // rank of this workgroup's load: 16 loads per pass, read four at a time so the reads overlap (entries past
      // pw hold INT_MAX and never count)
      int rk = 0;
      for (int u0 = 0; u0 < pw; u0 += 16) {
        int4 q[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) q[j] = *reinterpret_cast<const int4*>(&S.load[u0 + 4 * j]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int u = u0 + 4 * j;
          rk += (q[j].x < lm || (q[j].x == lm && u + 0 < m)) ? 1 : 0;
          rk += (q[j].y < lm || (q[j].y == lm && u + 1 < m)) ? 1 : 0;
          rk += (q[j].z < lm || (q[j].z == lm && u + 2 < m)) ? 1 : 0;
          rk += (q[j].w < lm || (q[j].w == lm && u + 3 < m)) ? 1 : 0;
        }
      }
      const int k = r * pw + rk;
      if (k < S.nreal) {
        int rank, head, level;
        vs_decode(S, H, x, k, rank, head, level);
        add = vs_cost(S, BM, G, rank, level);
        pos = k;
      }
    }
    __syncthreads();
    if (m < pw) {
      S.load[m] += add;
      if (m == me) S.mine[r] = pos;
    }
    __syncthreads();
  }
}

}  // namespace reax
