// Forward kernel for head_dim 128 (qpos and varlen masks, no gate epilogue) with 64 folded query rows per
// wavefront and the softmax interleaved with the MFMAs inside each wavefront. Same math and results contract as
// fmha_fwd_kernel (reference: libreax_howu/reax_fmha_v8.cu fmha3_kernel, causal / qpos visibility v8:155-162,
// 237), different schedule:
//   - One workgroup = 4 wavefronts (one per SIMD, up to 512 registers each) = 256 folded rows of one
//     (batch, KV head). A wavefront owns two 32-row blocks, so each K or V fragment it reads from LDS feeds two
//     MFMAs: half the LDS traffic per MFMA of a 32-row wavefront.
//   - Steady-state iteration i is one straight-line block of 32 MFMAs: O += V(i-1)^T P(i-1)^T (16) and
//     S(i+1)^T = K(i+1) Q^T (16), with the softmax of S(i) (computed one iteration earlier) into P(i) cut into
//     32 chunks, one after each MFMA. Measured on MI355X, a wavefront issues about five independent VALU
//     instructions under one of its own 32x32x16 MFMAs at no cost, and the softmax of a 32-key tile for 64 rows
//     is about that much per MFMA, so the VALU work hides under the matrix work.
//   - The MFMAs are inline assembly, ordered with the chunks by scheduling barriers: O accumulates in place in
//     the accumulation registers, Q is read from accumulation registers, S lands in VALU registers for the
//     softmax. (Left to itself the compiler alternates O between two register sets across the unrolled loop and
//     then copies Q and S between register files on every MFMA.) The compiler does not know these are MFMAs,
//     so results are read only after mfma_drain().
//   - S and P are double-buffered in registers; the loop is unrolled by two so the buffers keep fixed registers.
//   - The O rescale of the lazy online softmax (running max raised only when a row max grows by more than
//     RESCALE_SLACK in log2 units) is deferred to the iteration boundary: softmax(i) folds the factor into the
//     row sum at once and O is scaled before P(i) is accumulated, in a uniform branch that runs only when a
//     row's max actually grew.
//   - K/V tiles of 32 keys (two S and two P buffers and the K/V operands fit the 256 VALU registers) are loaded
//     straight into LDS two iterations (K) / one iteration (V) ahead, with one workgroup barrier per iteration.
#include "fmha_common.h"
#include "fmha_launch.h"
#include "fmha_tiles.h"

#include <climits>
#include <type_traits>

namespace reax {

constexpr int FA_NW = 4;           // wavefronts per workgroup, one per SIMD
constexpr int FA_BM = FA_NW * 64;  // folded rows per workgroup
constexpr int FA_BN = 32;          // keys per K/V tile
constexpr int FA_TILE = FA_BN * 128 * 2;
#ifndef REAX_FA_AHEAD
#define REAX_FA_AHEAD 5  // operand fragments read ahead of their MFMAs in the interleaved block
#endif
constexpr int FA_RING = 4;  // K/V ring slots: K is loaded 3 iterations ahead of its use, V 2 (see the pipeline)

#ifndef REAX_FA_NOPS
#define REAX_FA_NOPS ""
#endif
// O^T += V^T P^T block: accumulator in place in accumulation registers
__device__ __forceinline__ void mfma_o(f32x16_t& acc, const bf16x8_t& vf, const bf16x8_t& pb) {
  asm volatile(REAX_FA_NOPS "v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(vf), "v"(pb));
}
// S^T = K Q^T block: accumulator in VALU registers, Q operand from accumulation registers
__device__ __forceinline__ void mfma_s_first(f32x16_t& acc, const bf16x8_t& kf, const bf16x8_t& qa) {
  asm volatile(REAX_FA_NOPS "v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=v"(acc) : "v"(kf), "a"(qa));
}
__device__ __forceinline__ void mfma_s_acc(f32x16_t& acc, const bf16x8_t& kf, const bf16x8_t& qa) {
  asm volatile(REAX_FA_NOPS "v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(kf), "a"(qa));
}
// 3 x s_nop 7 = 24 wait states: more than a 32x32x16 MFMA's result needs before another instruction reads it
__device__ __forceinline__ void mfma_drain() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory"); }
// Self-guarding forms for code outside the interleaved block (prologue, epilogue): there the compiler may move
// accumulators between registers (v_accvgpr_mov) right next to an MFMA it does not know about, so each MFMA
// waits 5 states for operands written just before it and 24 after it before anything touches its result.
__device__ __forceinline__ void mfma_o_guarded(f32x16_t& acc, const bf16x8_t& vf, const bf16x8_t& pb) {
  asm volatile("s_nop 4\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
               : "+a"(acc) : "v"(vf), "v"(pb));
}
__device__ __forceinline__ void mfma_s_first_guarded(f32x16_t& acc, const bf16x8_t& kf, const bf16x8_t& qa) {
  asm volatile("s_nop 4\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, 0\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
               : "=v"(acc) : "v"(kf), "a"(qa));
}
__device__ __forceinline__ void mfma_s_acc_guarded(f32x16_t& acc, const bf16x8_t& kf, const bf16x8_t& qa) {
  asm volatile("s_nop 4\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
               : "+v"(acc) : "v"(kf), "a"(qa));
}
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }
// acc *= s for a block held in accumulation registers, one element at a time through one VALU register (a
// plain copy of the block to VALU registers would be hoisted by the compiler, needing 16 registers per block)
__device__ __forceinline__ void scale_acc(f32x16_t& acc, float s) {
  float t;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    float x = acc[e];
    asm volatile("v_accvgpr_read_b32 %1, %0\n\tv_mul_f32 %1, %1, %2\n\tv_accvgpr_write_b32 %0, %1"
                 : "+a"(x), "=&v"(t)
                 : "v"(s));
    acc[e] = x;
  }
}
// Redefines x in place (no instruction). Volatile statements keep their order, so touching a chunk's inputs right
// after its MFMA and its outputs before the next one confines the chunk's VALU work to that slot; scheduling
// barriers alone do not, as instruction selection already sinks side-effect-free arithmetic towards its uses.
__device__ __forceinline__ void pin(float& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void pin(uint32_t& x) { asm volatile("" : "+v"(x)); }
// element e of a block held in accumulation registers
__device__ __forceinline__ float acc_elem(const f32x16_t& acc, int e) {
  float x;
  asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(x) : "a"(acc[e]));
  return x;
}

template <int MODE>
__global__ void __launch_bounds__(256, 1) fmha_fwd_fa_kernel(const FwdParams p, int o_vec8) {
  constexpr int HD = 128;
  using T = FwdTile<HD>;
  __shared__ __align__(1024) uint8_t kring[FA_RING][FA_TILE];
  __shared__ __align__(1024) uint8_t vring[FA_RING][FA_TILE];
  __shared__ int s_lim[FA_NW];
  const int tid = threadIdx.x, lane = tid & 63, hf = lane >> 5, lr = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);

  // ---- workgroup -> (batch, KV head, row tile): heaviest tile first; when B*H % 8 == 0 each XCD (workgroups
  // are dealt to the 8 XCDs round-robin) serves a fixed set of KV heads from its own L2
  const int BH = p.B * p.H, id = blockIdx.x;
  int bh, rank;
  if ((BH & 7) == 0) {
    const int per = BH >> 3, x = id & 7, j = id >> 3;
    bh = x + 8 * (j % per);
    rank = j / per;
  } else {
    bh = id % BH;
    rank = id / BH;
  }
  const int tile = p.n_tiles - 1 - rank;
  const int b = bh / p.H, hk = bh - b * p.H;
  long long tok0 = 0;
  int Mb = p.M, Nb = p.N;
  if (MODE == MODE_VARLEN) {
    const int s0 = p.cu_seqlens[b], s1 = p.cu_seqlens[b + 1];
    tok0 = s0;
    Nb = s1 - s0;
    Mb = Nb * p.G;
  }
  const int r0 = tile * FA_BM;
  if (r0 >= Mb) return;  // uniform over the workgroup

  // ---- this lane's two query rows (row block rb: r0 + 64 w + 32 rb + lr) and their last visible keys
  int lim[2], tok[2], g[2];
  bool rvalid[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int r = r0 + 64 * w + 32 * rb + lr;
    rvalid[rb] = r < Mb;
    tok[rb] = rvalid[rb] ? r / p.G : 0;
    g[rb] = rvalid[rb] ? r - tok[rb] * p.G : 0;
    int l = -1;
    if (rvalid[rb]) {
      l = MODE == MODE_QPOS ? min(p.qpos[(long long)b * p.qpBs + tok[rb]], Nb - 1) : min(tok[rb], Nb - 1);
      l = max(l, -1);
    }
    lim[rb] = l;
  }
  const int wmax = __builtin_amdgcn_readfirstlane(wave_max(max(lim[0], lim[1])));
  const int wmin = __builtin_amdgcn_readfirstlane(wave_min(min(lim[0], lim[1])));
  if (lane == 0) s_lim[w] = wmax;
  __syncthreads();
  const int cmax = max(max(s_lim[0], s_lim[1]), max(s_lim[2], s_lim[3]));
  const int t_end = cmax < 0 ? 0 : cmax / FA_BN + 1;  // key tiles [0, t_end) of the workgroup

  // ---- Q fragments (B operand of S^T = K Q^T): dims 16 ks + 8 hf .. +7 of the lane's row in block rb
  bf16x8_t qf[2][T::QK];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const uint16_t* qrow = p.q + (long long)b * p.qsB + (long long)hk * p.qsH + (tok0 + tok[rb]) * p.qsT +
                           (long long)g[rb] * p.qsG;
#pragma unroll
    for (int ks = 0; ks < T::QK; ++ks) {
      const bf16x8_t qv = as_bf16x8(rvalid[rb] ? ld16(qrow + 16 * ks + 8 * hf) : u32x4_t{0u, 0u, 0u, 0u});
      asm volatile("" : "=a"(qf[rb][ks]) : "0"(qv));  // Q lives in accumulation registers from here on
    }
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_le(0));  // Q and qpos have landed before the (untracked) tile loads start
  const uint16_t* Kb = p.k + (long long)b * p.ksB + (long long)hk * p.ksH + tok0 * p.ksM;
  const uint16_t* Vb = p.v + (long long)b * p.vsB + (long long)hk * p.vsH + tok0 * p.vsM;
  const Dma<HD, FA_NW, FA_BN> kplan(p.ksM, w, lane), vplan(p.vsM, w, lane);
  const bool kfast = p.ksM * 2 * FA_BN < (1ll << 31), vfast = p.vsM * 2 * FA_BN < (1ll << 31);
  const uint32_t kbase = k_lane_base<HD>(0, lr, hf);
  const uint32_t vbase = v_lane_base<HD>(lane);

  f32x16_t o[2][T::DB];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int db = 0; db < T::DB; ++db) {
      f32x16_t z;
#pragma unroll
      for (int e = 0; e < 16; ++e) z[e] = 0.f;
      asm volatile("" : "=a"(o[rb][db]) : "0"(z));  // O lives in accumulation registers
    }
  float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f}, alpha_pend[2] = {1.f, 1.f};
  bool pend = false;  // wavefront-uniform: some row max grew since O was last rescaled
  const float cc = p.scale_log2;
  f32x16_t sA[2], sB[2];        // S^T buffers [row block]: s[rb][v] = score against key 8(v/4) + 4hf + v%4
  u32x4_t pA[2][2], pB[2][2];  // P buffers [row block][16-key step]: bf16 pairs 4ss..4ss+3, an MFMA operand each

  // operand fragments: V^T (dims 32db.., keys 16ss..) and K (keys 0..31, dims 16ks..)
  auto vfrag = [&](const uint8_t* vb_t, int ss, int db) __attribute__((always_inline)) {
    return v_operand<HD>(vb_t, db, ss, vbase);
  };
  auto kfrag = [&](const uint8_t* kb_t, int ks) __attribute__((always_inline)) {
    return as_bf16x8(*reinterpret_cast<const u32x4_t*>(kb_t + (kbase ^ (32u * ks))));
  };
  auto pfrag = [&](const u32x4_t (&pp)[2][2], int rb, int ss) __attribute__((always_inline)) {
    return as_bf16x8(pp[rb][ss]);
  };

  // plain (not interleaved) stages with self-guarding MFMAs, for the prologue and the epilogue
  auto qk = [&](const uint8_t* kb_t, f32x16_t (&sn)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int ks = 0; ks < T::QK; ++ks) {
      const bf16x8_t kf = kfrag(kb_t, ks);
      if (ks == 0) {
        mfma_s_first_guarded(sn[0], kf, qf[0][ks]);
        mfma_s_first_guarded(sn[1], kf, qf[1][ks]);
      } else {
        mfma_s_acc_guarded(sn[0], kf, qf[0][ks]);
        mfma_s_acc_guarded(sn[1], kf, qf[1][ks]);
      }
    }
  };
  auto pv = [&](const uint8_t* vb_t, const u32x4_t (&pp)[2][2]) __attribute__((always_inline)) {
#pragma unroll
    for (int ss = 0; ss < 2; ++ss)
#pragma unroll
      for (int db = 0; db < T::DB; ++db) {
        const bf16x8_t vf = vfrag(vb_t, ss, db);
        mfma_o_guarded(o[0][db], vf, pfrag(pp, 0, ss));
        mfma_o_guarded(o[1][db], vf, pfrag(pp, 1, ss));
      }
  };

  // ---- softmax pieces (row block rb of S^T in sc, P into pc)
  auto mask_rb = [&](int t, f32x16_t& s_rb, int rb) __attribute__((always_inline)) {
    // key t*BN + 8(v/4) + 4hf + v%4 is visible iff 8(v/4) + v%4 <= lim - t*BN - 4hf
    const int d = lim[rb] - t * FA_BN - 4 * hf;
#pragma unroll
    for (int v = 0; v < 16; ++v)
      if (8 * (v >> 2) + (v & 3) > d) s_rb[v] = -INFINITY;
  };
  // running-max update of row block rb from its tile max mx (log2 units); returns the exponent offset
  auto update_rb = [&](int rb, float mx) __attribute__((always_inline)) {
    const bool grow = __any(mx > m_run[rb] + RESCALE_SLACK);
    const float m_new = grow ? fmaxf(m_run[rb], mx) : m_run[rb];
    const float alpha = m_new == m_run[rb] ? 1.0f : fast_exp2(m_run[rb] - m_new);
    l_run[rb] *= alpha;
    alpha_pend[rb] *= alpha;
    pend = pend || grow;
    m_run[rb] = m_new;
    return m_new == -INFINITY ? 0.f : m_new;
  };
  auto softmax_plain = [&](int t, f32x16_t (&sc)[2], u32x4_t (&pc)[2][2]) __attribute__((always_inline)) {
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      mask_rb(t, sc[rb], rb);
      float mx = -INFINITY;
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = fmaxf(mx, sc[rb][v]);
      const float m_use = update_rb(rb, halves_max(mx) * cc);
      float ps[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float p0 = fast_exp2(__builtin_fmaf(sc[rb][2 * i], cc, -m_use));
        const float p1 = fast_exp2(__builtin_fmaf(sc[rb][2 * i + 1], cc, -m_use));
        ps[(i & 1) * 2] += p0;
        ps[(i & 1) * 2 + 1] += p1;
        pc[rb][i >> 2][i & 3] = pack_bf16x2(p0, p1);
      }
      l_run[rb] += (ps[0] + ps[1]) + (ps[2] + ps[3]);
    }
  };

  // ---- the interleaved block of iteration t: PV(t-1) from vread with pp, QK(t+1) from kread into sn,
  // softmax(t) of sc into pc. Slot k (0..31) = MFMA k, then the LDS reads of the fragment three ahead, then
  // VALU chunk k:
  //   slots 0-3 row maxima, 4 the half-wavefront max, 5-6 the running-max updates, 7-31 the exponentials of
  //   the 16 element pairs (pair j: fma in slot 7 + 3j/2, exp one slot later, sum and bf16 pack one more).
  // MFMA k < 16: O[rb = k&1][db = (k>>1)&3] with V fragment f = k>>1 (ss = f>>2, db = f&3);
  // MFMA k >= 16: S[rb = k&1] with K fragment f = k>>1 (ks = f - 8).
  auto fused = [&](int t, const uint8_t* vread, const uint8_t* kread, f32x16_t (&sc)[2], f32x16_t (&sn)[2],
                   u32x4_t (&pc)[2][2], const u32x4_t (&pp)[2][2], bool masked) __attribute__((always_inline)) {
    constexpr int AHEAD = REAX_FA_AHEAD;
    bf16x8_t frag[16];
    bf16x8_t pb[2][2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int ss = 0; ss < 2; ++ss) pb[rb][ss] = pfrag(pp, rb, ss);
    auto load = [&](int f) __attribute__((always_inline)) {
      if (f < 8)
        frag[f] = vfrag(vread, f >> 2, f & 3);
      else
        frag[f] = kfrag(kread, f - 8);
    };
#pragma unroll
    for (int f = 0; f < AHEAD; ++f) load(f);
    if (masked) {
      mask_rb(t, sc[0], 0);
      mask_rb(t, sc[1], 1);
    }
    float mp[2][4], mx[2], m_use[2], ps[2][4];
    float pe[2][16];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int j = 0; j < 4; ++j) ps[rb][j] = 0.f;
    static_for<0, 32>([&](auto kc) __attribute__((always_inline)) {
      constexpr int k = decltype(kc)::value;
      constexpr int f = k >> 1, rb = k & 1;
      sched_fence();
      if constexpr (k < 16)
        mfma_o(o[rb][f & 3], frag[f], pb[rb][f >> 2]);
      else if constexpr (k < 18)
        mfma_s_first(sn[rb], frag[f], qf[rb][f - 8]);
      else
        mfma_s_acc(sn[rb], frag[f], qf[rb][f - 8]);
      sched_fence();
      if constexpr ((k & 1) == 0 && f + AHEAD < 16) load(f + AHEAD);
      // VALU chunk k
      if constexpr (k == 0) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          mp[r][0] = __builtin_fmaxf(__builtin_fmaxf(sc[r][0], sc[r][1]), sc[r][2]);
          mp[r][1] = __builtin_fmaxf(__builtin_fmaxf(sc[r][3], sc[r][4]), sc[r][5]);
          pin(mp[r][0]);
          pin(mp[r][1]);
        }
      } else if constexpr (k == 1) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          mp[r][2] = __builtin_fmaxf(__builtin_fmaxf(sc[r][6], sc[r][7]), sc[r][8]);
          mp[r][3] = __builtin_fmaxf(__builtin_fmaxf(sc[r][9], sc[r][10]), sc[r][11]);
          pin(mp[r][2]);
          pin(mp[r][3]);
        }
      } else if constexpr (k == 2) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          mp[r][0] = __builtin_fmaxf(__builtin_fmaxf(mp[r][0], sc[r][12]), sc[r][13]);
          mp[r][1] = __builtin_fmaxf(__builtin_fmaxf(mp[r][1], sc[r][14]), sc[r][15]);
          pin(mp[r][0]);
          pin(mp[r][1]);
        }
      } else if constexpr (k == 3) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          mx[r] = __builtin_fmaxf(__builtin_fmaxf(mp[r][0], mp[r][1]), __builtin_fmaxf(mp[r][2], mp[r][3]));
          pin(mx[r]);
        }
      } else if constexpr (k == 4) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          mx[r] = halves_max(mx[r]) * cc;
          pin(mx[r]);
        }
      } else if constexpr (k == 5 || k == 6) {
        m_use[k - 5] = update_rb(k - 5, mx[k - 5]);
        pin(m_use[k - 5]);
        pin(l_run[k - 5]);
      } else {
        // pair j = (row block j&1, pair index j>>1): fma in slot 7 + 3j/2, exp +1, sum + pack +2
        static_for<0, 16>([&](auto jc) __attribute__((always_inline)) {
          constexpr int j = decltype(jc)::value;
          constexpr int s0 = 7 + (3 * j) / 2, r = j & 1, i = j >> 1;
          if constexpr (k == s0) {
            float a0 = sc[r][2 * i], a1 = sc[r][2 * i + 1];
            pin(a0);
            pin(a1);
            pe[r][2 * i] = __builtin_fmaf(a0, cc, -m_use[r]);
            pe[r][2 * i + 1] = __builtin_fmaf(a1, cc, -m_use[r]);
            pin(pe[r][2 * i]);
            pin(pe[r][2 * i + 1]);
          } else if constexpr (k == s0 + 1) {
            pe[r][2 * i] = fast_exp2(pe[r][2 * i]);
            pe[r][2 * i + 1] = fast_exp2(pe[r][2 * i + 1]);
            pin(pe[r][2 * i]);
            pin(pe[r][2 * i + 1]);
          } else if constexpr (k == s0 + 2) {
            ps[r][(i & 1) * 2] += pe[r][2 * i];
            ps[r][(i & 1) * 2 + 1] += pe[r][2 * i + 1];
            uint32_t pk = pack_bf16x2(pe[r][2 * i], pe[r][2 * i + 1]);
            pin(ps[r][(i & 1) * 2]);
            pin(ps[r][(i & 1) * 2 + 1]);
            pin(pk);
            pc[r][i >> 2][i & 3] = pk;
          }
        });
      }
    });
    sched_fence();
#pragma unroll
    for (int r = 0; r < 2; ++r) l_run[r] += (ps[r][0] + ps[r][1]) + (ps[r][2] + ps[r][3]);
  };

  // O *= alpha_pend (rows whose max grew), before the next P is accumulated; O is still zero before the first
  // P.V, so then only the factors are reset. One 16-register block at a time through VALU registers.
  auto rescale = [&](bool o_live) __attribute__((always_inline)) {
    if (pend) {
      if (o_live) {
        mfma_drain();
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
          for (int db = 0; db < T::DB; ++db) scale_acc(o[rb][db], alpha_pend[rb]);
        mfma_drain();
      }
      alpha_pend[0] = alpha_pend[1] = 1.f;
      pend = false;
    }
  };

  // Software pipeline over key tiles. Iteration i (1 <= i < t_end) reads K(i+1) (QK) from kring[(i+1)%4] and
  // V(i-1) (PV) from vring[(i-1)%4], and loads K(i+4) into kring[i%4] and V(i+2) into vring[(i+2)%4]: slots last
  // read in iteration i-1. At its end K(i+2) and V(i), loaded two iterations earlier, must have landed: the loads
  // of iterations i-1 and i may stay in flight (loads return in order). In the last iteration QK(t_end) reads a
  // stale but in-bounds K slot and its S is never used. The prologue loads K(0..3), V(0..2), does QK(0), loads
  // K(4), then softmax(0) and QK(1); the epilogue PV(t_end-1). Ring slots and the S/P buffer parity follow i, so
  // the loop body is written for each i mod 4.
  constexpr int KL = Dma<HD, FA_NW, FA_BN>::DW;  // direct-to-LDS loads per wavefront per K or V tile
  auto loads_of = [&](int i) __attribute__((always_inline)) {
    // loads this wavefront issued in iteration i (the prologue's K(4) counts as iteration 0's)
    return (i + 4 < t_end ? KL : 0) + (i >= 1 && i + 2 < t_end ? KL : 0);
  };
  auto wait_loads = [&](int in_flight) __attribute__((always_inline)) {
    // s_waitcnt needs an immediate: in_flight is one of 0, KL, .., 4 KL
    if (in_flight >= 4 * KL)
      __builtin_amdgcn_s_waitcnt(vmcnt_le(4 * KL));
    else if (in_flight == 3 * KL)
      __builtin_amdgcn_s_waitcnt(vmcnt_le(3 * KL));
    else if (in_flight == 2 * KL)
      __builtin_amdgcn_s_waitcnt(vmcnt_le(2 * KL));
    else if (in_flight == KL)
      __builtin_amdgcn_s_waitcnt(vmcnt_le(KL));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_le(0));
  };
  auto iteration = [&](int i, auto rc) __attribute__((always_inline)) {
    constexpr int R = decltype(rc)::value;  // i % 4
    constexpr bool odd = R & 1;
    f32x16_t(&sc)[2] = odd ? sB : sA;
    f32x16_t(&sn)[2] = odd ? sA : sB;
    u32x4_t(&pc)[2][2] = odd ? pB : pA;
    u32x4_t(&pp)[2][2] = odd ? pA : pB;
    const uint8_t* kread = kring[(R + 1) % FA_RING];
    const uint8_t* vread = vring[(R + 3) % FA_RING];
    rescale(i >= 2);
    if (i + 4 < t_end) kplan.template tile<1>(kring[R], Kb, p.ksM, kfast, (i + 4) * FA_BN, Nb, w, lane);
    if (i + 2 < t_end) vplan.template tile<1>(vring[(R + 2) % FA_RING], Vb, p.vsM, vfast, (i + 2) * FA_BN, Nb, w, lane);
#ifdef REAX_FA_PLAIN
    pv(vread, pp);
    qk(kread, sn);
    mfma_drain();
    softmax_plain(i, sc, pc);
#else
    fused(i, vread, kread, sc, sn, pc, pp, i * FA_BN + FA_BN - 1 > wmin);
#endif
    mfma_drain();                               // S(i+1) is read by the next iteration's softmax
    wait_loads(loads_of(i - 1) + loads_of(i));  // K(i+2), V(i) have landed (this wavefront's part)
    // ... and every other wavefront's, and all LDS reads of this iteration are done. Not __syncthreads(): its
    // fence waits for every load in flight (vmcnt(0)), i.e. also for the tiles of the next two iterations.
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };

  if (t_end > 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (j < t_end) kplan.template tile<1>(kring[j], Kb, p.ksM, kfast, j * FA_BN, Nb, w, lane);
#pragma unroll
    for (int j = 0; j < 3; ++j)
      if (j < t_end) vplan.template tile<1>(vring[j], Vb, p.vsM, vfast, j * FA_BN, Nb, w, lane);
    __builtin_amdgcn_s_waitcnt(vmcnt_le(0));
    __syncthreads();
    qk(kring[0], sA);
    mfma_drain();
    __syncthreads();  // K(0) is read by every wavefront before K(4) is loaded over it
    if (4 < t_end) kplan.template tile<1>(kring[0], Kb, p.ksM, kfast, 4 * FA_BN, Nb, w, lane);
    if (t_end > 1) qk(kring[1], sB);
    sched_fence();
    softmax_plain(0, sA, pA);
    sched_fence();
    mfma_drain();
    __syncthreads();  // (K(2), V(0) landed before the first barrier)
    for (int i = 1; i < t_end; i += 4) {
      iteration(i, std::integral_constant<int, 1>{});
      if (i + 1 < t_end) iteration(i + 1, std::integral_constant<int, 2>{});
      if (i + 2 < t_end) iteration(i + 2, std::integral_constant<int, 3>{});
      if (i + 3 < t_end) iteration(i + 3, std::integral_constant<int, 0>{});
    }
    rescale(t_end >= 2);
    // PV(t_end-1): P in the buffer of parity (t_end-1), V in vring[(t_end-1)%4]
    const bool last_odd = (t_end - 1) & 1;
    u32x4_t pl[2][2];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int ss = 0; ss < 2; ++ss) pl[rb][ss] = last_odd ? pB[rb][ss] : pA[rb][ss];
    pv(vring[(t_end - 1) & (FA_RING - 1)], pl);
    mfma_drain();
  }

  // ---- epilogue: normalise, LSE, store (O^T layout: lane holds dims 32db + 8(v/4) + 4hf + v%4 of its row)
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const float l = halves_sum(l_run[rb]);
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    if (!rvalid[rb]) continue;
    if (p.lse && hf == 0) {
      const float lse = l > 0.f ? (m_run[rb] + log2f(l)) * 0.69314718055994530942f : -INFINITY;
      p.lse[(long long)b * p.lsB + (long long)hk * p.lsH + (tok0 + tok[rb]) * p.lsT + (long long)g[rb] * p.lsG] = lse;
    }
    if (!p.o) continue;
    uint16_t* orow =
        p.o + (long long)b * p.osB + (long long)hk * p.osH + (tok0 + tok[rb]) * p.osT + (long long)g[rb] * p.osG;
#pragma unroll
    for (int db = 0; db < T::DB; ++db) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d = 32 * db + 8 * q4 + 4 * hf;
        const uint32_t w0 = pack_bf16x2(acc_elem(o[rb][db], 4 * q4 + 0) * inv, acc_elem(o[rb][db], 4 * q4 + 1) * inv);
        const uint32_t w1 = pack_bf16x2(acc_elem(o[rb][db], 4 * q4 + 2) * inv, acc_elem(o[rb][db], 4 * q4 + 3) * inv);
        if (o_vec8) {
          *reinterpret_cast<u32x2_t*>(orow + d) = u32x2_t{w0, w1};
        } else {
          *reinterpret_cast<uint32_t*>(orow + d) = w0;
          *reinterpret_cast<uint32_t*>(orow + d + 2) = w1;
        }
      }
    }
  }
}

int launch_fwd_fa(const FwdParams& p0, int mode, int o_vec8, hipStream_t stream) {
  FwdParams p = p0;
  p.n_tiles = (int)(((long long)p.M + FA_BM - 1) / FA_BM);
  const long long nwg = (long long)p.B * p.H * p.n_tiles;
  if (nwg <= 0 || nwg > INT_MAX) return (int)hipErrorInvalidConfiguration;
  if (mode == MODE_QPOS)
    hipLaunchKernelGGL(fmha_fwd_fa_kernel<MODE_QPOS>, dim3((unsigned)nwg), dim3(64 * FA_NW), 0, stream, p, o_vec8);
  else if (mode == MODE_VARLEN)
    hipLaunchKernelGGL(fmha_fwd_fa_kernel<MODE_VARLEN>, dim3((unsigned)nwg), dim3(64 * FA_NW), 0, stream, p, o_vec8);
  else
    return (int)hipErrorInvalidValue;
  return (int)hipGetLastError();
}

}  // namespace reax
