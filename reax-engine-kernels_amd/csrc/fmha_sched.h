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
//   4. batched longest-processing-time assignment within the class: round 0 hands the class's first PW items to
//      its PW workgroups in turn; every later round hands the next PW / 2 items to the PW / 2 workgroups holding
//      the least work (in increasing order of that work, ties by index).
// Steps 1-3 build tables (the class's pairs, their prefix sums, the level starts, and each item's identity and
// cost) with every thread of the workgroup, and the rounds run in one wavefront, each a rank scan of the loads
// (kept as distinct keys, load * 256 + index) and one table read. Round 0's item follows from the tables alone, so
// the kernel issues that item's first loads before the rounds and runs them while the loads are in flight. On config 3 (stamped copy of the kernel) the
// schedule takes ~5.8 us before the first item, against ~7 us when each round decoded its items and compared
// (load, index) pairs, and the busiest workgroup's items ~54 us, against ~56 us when every round handed out PW
// items (half rounds get as close as one-item-at-a-time LPT, in a few rounds): 0.0722 -> 0.0677 ms.
// Shapes beyond the LDS tables (VS_NSEQ sequences, VS_NPAIR pairs per class, VS_TMAX tiles per sequence,
// VS_KTAB items per class, VS_PMAX workgroups, VS_RMAX rounds) keep the fixed order.
#pragma once
#include <climits>

#include "fmha_common.h"

namespace reax {

constexpr int VS_NSEQ = 256, VS_NPAIR = 256, VS_TMAX = 1024, VS_KTAB = 1024, VS_PMAX = 256, VS_RMAX = 64;

struct VarlenSched {
  int sorted[VS_NSEQ];     // sequence index by rank (most items first)
  int Ts[VS_NSEQ];         // items of the sequence of each rank
  int pbh[VS_NPAIR];       // the class's pairs in deal order: sequence * H + KV head
  int pT[VS_NPAIR];        //   their item counts (never increasing along the order)
  int pL[VS_NPAIR];        //   their tokens
  int pref[VS_NPAIR + 1];  // prefix sums of pT
  int start[VS_TMAX];      // first position of level i in the class's item order
  int kitem[VS_KTAB];      // item at position k of the order: its pair's sequence * H + KV head, times 1024, plus level
  int kcost[VS_KTAB];      // its cost (half tile-steps)
  alignas(16) int load[VS_PMAX];  // work held by class workgroup m (half tile-steps) * 256 + m; INT_MAX past pw
  int mine[VS_RMAX];       // this workgroup's item (as kitem) from round r, -1 for none
  int ok, tmax, nreal, rounds, npc;
};

// k-th pair of class x of nx (snake deal): pairs 0..nx-1 go to classes 0..nx-1, pairs nx..2nx-1 to nx-1..0, ...
__device__ __forceinline__ int vs_pair(int k, int x, int nx) {
  return 2 * nx * (k >> 1) + ((k & 1) ? 2 * nx - 1 - x : x);
}

// Inclusive prefix sum over the wavefront's lanes: within each 16-lane row by DPP shifts (lane i adds lanes i - 1,
// then i - 2 .. i - 3, i - 4 .. i - 7, i - 8 .. i - 15 of the partial sums), across rows by the row broadcasts of
// lane 15 into rows 1 and 3 and of lane 31 into rows 2 and 3.
__device__ __forceinline__ int wave_scan_add(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15 into rows 1, 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31 into rows 2, 3
  return x;
}

// Cost of an item in half tile-steps: its key tiles plus a fixed per-item overhead (prologue and epilogue, which
// measured ~2.8 key tiles' time on config 3). tpl = tokens per level (BM / G), L = the sequence's tokens.
__device__ __forceinline__ int vs_cost(int tpl, int L, int level) {
  const int last = min((level + 1) * tpl, L) - 1;
  return 2 * (last / 64 + 1) + 5;
}

// Builds the schedule's tables (every thread of the workgroup calls it; it ends with a barrier). Sets S.ok = 0 when
// the shape exceeds the tables. wg is the workgroup index, P the grid size. With S.ok set, this workgroup's round-0
// item is vs_first(S, P, wg) right away; vs_rounds then fills S.mine[].
template <int BM>
__device__ void vs_build(VarlenSched& S, const int* cu, int nseq, int H, int G, int P, int wg) {
  const int tid = threadIdx.x, nt = blockDim.x;
  if (nseq > VS_NSEQ || P > VS_PMAX || nseq <= 0 || H <= 0 || BM % G != 0 || (long long)nseq * H > INT_MAX / 1024) {
    if (tid == 0) S.ok = 0;
    __syncthreads();
    return;
  }
  const int nx = (P % 8 == 0) ? 8 : 1, x = wg % nx, pw = P / nx, me = wg / nx, tpl = BM / G;
  // the class's pair count: pairs 2 nx i + x and 2 nx i + 2 nx - 1 - x below nseq * H, a prefix of the deal
  const long long npairs = (long long)nseq * H, full = npairs / (2 * nx), rem = npairs - full * 2 * nx;
  const long long npc_l = 2 * full + (rem > x ? 1 : 0) + (rem > 2 * nx - 1 - x ? 1 : 0);
  if (npc_l > VS_NPAIR) {
    if (tid == 0) S.ok = 0;
    __syncthreads();
    return;
  }
  const int npc = (int)npc_l;
  // items and tokens per sequence, staged in kitem[] and start[] (VS_KTAB, VS_TMAX >= VS_NSEQ): cu_seqlens is
  // read once
  for (int s = tid; s < nseq; s += nt) {
    const int L = cu[s + 1] - cu[s];
    S.kitem[s] = L > 0 ? (int)(((long long)L * G + BM - 1) / BM) : 0;
    S.start[s] = L;
  }
  __syncthreads();
  for (int s = tid; s < nseq; s += nt) {
    const int T = S.kitem[s];
    int r = 0;
    for (int u = 0; u < nseq; ++u) {
      const int Tu = S.kitem[u];
      r += (Tu > T || (Tu == T && u < s)) ? 1 : 0;
    }
    S.sorted[r] = s;
    S.Ts[r] = T;
  }
  __syncthreads();
  if (tid < 64) {
    // wavefront 0: the class's pairs in deal order (lane l takes pairs 4 l .. 4 l + 3; VS_NPAIR = 256) and the
    // prefix sums of their item counts (a scan over the lanes' sums)
    const int lane = tid;
    int v[4], sum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = 4 * lane + i;
      v[i] = 0;
      if (q < npc) {
        const int j = vs_pair(q, x, nx), rank = j / H, head = j - rank * H, s = S.sorted[rank];
        v[i] = S.Ts[rank];
        S.pbh[q] = s * H + head;
        S.pT[q] = v[i];
        S.pL[q] = S.start[s];
      }
      sum += v[i];
    }
    const int incl = wave_scan_add(sum);
    int acc = incl - sum;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (4 * lane + i <= npc) S.pref[4 * lane + i] = acc;
      acc += v[i];
    }
    if (lane == 63) {
      if (npc == VS_NPAIR) S.pref[VS_NPAIR] = incl;
      const int nreal = incl, tmax = npc > 0 ? S.Ts[vs_pair(0, x, nx) / H] : 0, hb = max(1, pw / 2);
      const int rounds = nreal <= pw ? (nreal > 0 ? 1 : 0) : 1 + (nreal - pw + hb - 1) / hb;
      S.npc = npc;
      S.tmax = tmax;
      S.nreal = nreal;
      S.rounds = rounds;
      // the rounds key a load by load * 256 + index: the class's whole work must stay below 2^23
      const long long most = (long long)nreal * (2 * ((long long)tmax * tpl / 64 + 1) + 5);
      S.ok = (tmax <= VS_TMAX && nreal <= VS_KTAB && rounds <= VS_RMAX && most < (1ll << 23)) ? 1 : 0;
    }
  }
  __syncthreads();
  if (!S.ok) return;
  const int tmax = S.tmax, nreal = S.nreal;
  // start[i] = items on levels above i = sum over the c pairs reaching level i + 1 of (items - (i + 1)); those
  // pairs are a prefix of the class's pair list (item counts never increase along it)
  for (int i = tid; i < tmax; i += nt) {
    int lo = 0, hi = npc;  // c = the first pair with at most i + 1 items
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (S.pT[mid] > i + 1) lo = mid + 1; else hi = mid;
    }
    S.start[i] = S.pref[lo] - lo * (i + 1);
  }
  for (int m = tid; m < VS_PMAX; m += nt) S.load[m] = m < pw ? m : INT_MAX;
  for (int r = tid; r < VS_RMAX; r += nt) S.mine[r] = -1;
  __syncthreads();
  // each item's identity and cost: start[] decreases as the level rises and level i holds positions
  // [start[i], start[i - 1]), so item k's level is the lowest one whose start is <= k
  for (int k = tid; k < nreal; k += nt) {
    int lo = 0, hi = tmax - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (S.start[mid] <= k) hi = mid; else lo = mid + 1;
    }
    const int q = k - S.start[lo];
    S.kitem[k] = S.pbh[q] * 1024 + lo;
    S.kcost[k] = vs_cost(tpl, S.pL[q], lo);
  }
  __syncthreads();
}

// This workgroup's item from round 0 (as kitem, -1 for none): every load starts at zero work, so the rank of class
// workgroup m's key (0 * 256 + m) is m, and round 0 gives it item m.
__device__ __forceinline__ int vs_first(const VarlenSched& S, int P, int wg) {
  const int me = wg / ((P % 8 == 0) ? 8 : 1);
  return me < S.nreal ? S.kitem[me] : -1;
}

// The rounds, in wavefront 0 alone (every thread may call it; threads of the other wavefronts return at once). Its
// LDS accesses complete in issue order, so no barrier is needed between a round's reads and writes; the caller
// puts a workgroup barrier between this call and any read of S.mine[]. Needs the tables of vs_build with S.ok set.
__device__ void vs_rounds(VarlenSched& S, int P, int wg) {
  const int tid = threadIdx.x;
  const int nx = (P % 8 == 0) ? 8 : 1, pw = P / nx, me = wg / nx, nreal = S.nreal;
  if (tid < 64) {
    // lane l stands for class workgroups l, l + 64, l + 128, l + 192
    const int lane = tid, hb = max(1, pw / 2), rounds = S.rounds;
    for (int r = 0; r < rounds; ++r) {
      const int base = r == 0 ? 0 : pw + (r - 1) * hb, batch = r == 0 ? pw : hb;
      int add[VS_PMAX / 64], pos[VS_PMAX / 64];
#pragma unroll
      for (int i = 0; i < VS_PMAX / 64; ++i) {
        const int m = lane + 64 * i;
        add[i] = 0;
        pos[i] = -1;
        if (m < pw) {
          // rank of this workgroup's load: the keys (load * 256 + index) are distinct, so it is the count of
          // smaller keys; 16 per pass, read four at a time so the reads overlap
          const int lm = S.load[m];
          int rk = 0;
          for (int u0 = 0; u0 < pw; u0 += 16) {
            int4 qv[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) qv[j] = *reinterpret_cast<const int4*>(&S.load[u0 + 4 * j]);
#pragma unroll
            for (int j = 0; j < 4; ++j)
              rk += (qv[j].x < lm ? 1 : 0) + (qv[j].y < lm ? 1 : 0) + (qv[j].z < lm ? 1 : 0) + (qv[j].w < lm ? 1 : 0);
          }
          const int k = base + rk;
          if (rk < batch && k < nreal) {
            add[i] = S.kcost[k];
            pos[i] = S.kitem[k];
          }
        }
      }
      asm volatile("" ::: "memory");  // the round's reads stay before its writes
#pragma unroll
      for (int i = 0; i < VS_PMAX / 64; ++i) {
        const int m = lane + 64 * i;
        if (m < pw) {
          S.load[m] += add[i] << 8;
          if (m == me) S.mine[r] = pos[i];
        }
      }
      asm volatile("" ::: "memory");  // and its writes before the next round's reads
    }
  }
}

}  // namespace reax
