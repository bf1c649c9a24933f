// Attention forward for head_dim 256 on gfx950: the shape of the drop-in entry points (reax_fmha_q / reax_fmha_qp,
// reference: libreax_howu/reax_fmha_v8.cu:115-450 and libreax_fmha_post/reax_fmha_v11.cu:172-590, HD 256).
//
// A 32-row block at head_dim 256 needs 128 fp32 registers of O and 64 of Q per lane, which leaves no room for two
// wavefronts per SIMD. Here a *pair* of wavefronts shares each 32-row block, split along both products:
//   - S = Q K^T: wavefront `role` 0 computes the scores of keys 0..31 of every 64-key tile, role 1 keys 32..63,
//     each over all 256 dims (Q stays in registers: 64 VGPRs);
//   - O = P V: role 0 accumulates dims 0..127, role 1 dims 128..255, each over all 64 keys of the tile.
// The pair exchanges two things through LDS per tile: its row maxima (32 floats, so both use the tile's max) and
// its bf16 probabilities (2 KB, the other half of P for P.V). Per wavefront and tile that is 16 + 16 MFMAs
// (v_mfma_f32_32x32x16_bf16) and 16 softmax elements per lane: O 64 + Q 64 + S 16 + P 8 registers, two wavefronts
// per SIMD.
//
// Workgroup = 8 wavefronts = 2 groups x 2 pairs x 2 roles = 128 folded rows. Wavefronts w and w + 4 share a SIMD
// (the dispatcher deals a workgroup's wavefronts round-robin over the CU's 4 SIMDs), and the groups ping-pong as in
// the head_dim-128 kernel:
//     half 1 of step t: group 0 runs its MFMA phase  [S(t) = Q K(t)^T, then O += P(t-1) V(t-1)]
//                       group 1 runs its VALU phase  [softmax of S(t-1), then the K(t+1) tile loads]
//     half 2 of step t: group 1 runs its MFMA phase, group 0 the V(t) tile loads and the softmax of S(t).
// The row maxima of S(t) are computed at the end of the MFMA phase (while the P.V MFMAs run) and published at the
// next barrier; the probabilities at the end of the softmax phase, for the partner's next MFMA phase. The softmax
// phase is about half as long as an MFMA phase, so the direct-to-LDS tile loads (64 KB per step) are issued from
// the softmax phases, where they cost no matrix-core time: K(t+1) by group 1 at the start of half 1, V(t) by group
// 0 at the start of half 2; the MFMA phases run at a raised wave priority.
// (Issued all in half 1, with group 1's softmax, they made that half longer than the MFMA phase opposite it:
// config 5 ran 9.9 ms that way and 8.65 ms split.)
#include "fmha_common.h"
#include "fmha_launch.h"
#include "fmha_tiles.h"

#include <climits>
#include <type_traits>

namespace reax {

constexpr int PR_NW = 8;    // wavefronts per workgroup
constexpr int PR_BM = 128;  // folded rows per workgroup item

template <int MODE, bool POST>
__global__ void __launch_bounds__(512, 1) fmha_fwd_pair_kernel(const FwdParams p, int o_vec8) {
  constexpr int HD = 256;
  using T = FwdTile<HD>;  // 64-key tiles of 32 KB; QK = 16 k-steps over the head dim
  constexpr int NDB = 4;  // 32-dim blocks of O per wavefront (its half of the head dim)
  __shared__ __align__(1024) uint8_t kring[2][T::TILE];
  __shared__ __align__(1024) uint8_t vring[2][T::TILE];
  __shared__ __align__(16) u32x4_t xp[PR_NW][2][64];  // bf16 P of a wavefront's 32 keys, in B-operand lane order
  __shared__ float xm[PR_NW][32];                      // row max of a wavefront's 32 keys of the current tile
  __shared__ float xl[PR_NW][32];                      // row sums (epilogue)
  __shared__ int s_lim[PR_NW];
  __shared__ int s_raw[PR_NW];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, hf = lane >> 5, lr = lane & 31;
  const int grp = w >> 2, pair = (w >> 1) & 1, role = w & 1, partner = w ^ 1;
  const uint32_t gu = __builtin_amdgcn_readfirstlane(w & 3);  // index within the group, as a scalar

  const int BH = p.B * p.H;
  const long long n_items = (long long)BH * p.n_tiles;
  const bool xcd_aware = MODE != MODE_VARLEN && (BH & 7) == 0 && (gridDim.x & 7) == 0;
  auto item = [&](int id) __attribute__((always_inline)) {
    int bh, rank;
    if (xcd_aware) {
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
    const int r0 = tile * PR_BM;
    if (r0 >= Mb) return;  // uniform over the workgroup

    const int r = r0 + 64 * grp + 32 * pair + lr;
    const bool rvalid = r < Mb;
    const int tok = rvalid ? r / p.G : 0;
    const int g = rvalid ? r - tok * p.G : 0;
    int lim = -1, qraw = -1;
    if (rvalid) {
      if (MODE == MODE_QPOS) {
        qraw = p.qpos[(long long)b * p.qpBs + tok];
        lim = min(qraw, Nb - 1);
      } else {
        lim = min(tok, Nb - 1);
      }
      lim = max(lim, -1);
    }
    const bool blk0 = MODE == MODE_QPOS && p.qpos0_block;
    int wmax = wave_max(lim), wmin = wave_min(lim);
    if (blk0) {
      const int rmax = wave_max(qraw);
      if (lane == 0) s_raw[w] = rmax;
    }
    if (lane == 0) s_lim[w] = wmax;
    __syncthreads();
    if (blk0) {
      // the reference's 64-row blocks: a group's four wavefronts (two pairs) hold rows [r0 + 64 grp, +64), and
      // r0 is a multiple of 128; a block whose largest raw qpos is 0 stores V[0] in every live row
      const int bmax = max(max(s_raw[4 * grp], s_raw[4 * grp + 1]), max(s_raw[4 * grp + 2], s_raw[4 * grp + 3]));
      if (bmax == 0 && rvalid && Nb > 0) lim = 0;
      wmax = wave_max(lim);
      wmin = wave_min(lim);
    }
    int cmax = s_lim[0];
#pragma unroll
    for (int i = 1; i < PR_NW; ++i) cmax = max(cmax, s_lim[i]);
    const int t_end = cmax < 0 ? 0 : cmax / T::BN + 1;

    const uint16_t* qrow = p.q + (long long)b * p.qsB + (long long)hk * p.qsH + (tok0 + tok) * p.qsT + (long long)g * p.qsG;
    bf16x8_t qf[T::QK];
#pragma unroll
    for (int ks = 0; ks < T::QK; ++ks)
      qf[ks] = as_bf16x8(rvalid ? ld16(qrow + 16 * ks + 8 * hf) : u32x4_t{0u, 0u, 0u, 0u});
    const uint16_t* Kb = p.k + (long long)b * p.ksB + (long long)hk * p.ksH + tok0 * p.ksM;
    const uint16_t* Vb = p.v + (long long)b * p.vsB + (long long)hk * p.vsH + tok0 * p.vsM;

    f32x16_t o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[db][e] = 0.f;
    float m_run = -INFINITY, l_run = 0.f, m_own = -INFINITY;
    const float cc = p.scale_log2;
    f32x16_t s;
    uint32_t pk[8];

    const bool kfast = p.ksM * 2 * T::BN < (1ll << 31), vfast = p.vsM * 2 * T::BN < (1ll << 31);
    const uint32_t kbase = k_lane_base<HD>(role, lr, hf);
    const uint32_t vbase = v_lane_base<HD>(lane);

    // softmax of tile t (S(t) masked in s, this wavefront's row max in m_own, the partner's in xm): P -> pk and
    // xp[w], running max / row sum of this wavefront's keys, lazy O rescale
    auto softmax = [&](int t) __attribute__((always_inline)) {
      if (t * T::BN > wmax) return;
      const float mx = fmaxf(m_own, xm[partner][lr]);  // both wavefronts of the pair get the same tile max
      if (__any(mx > m_run + RESCALE_SLACK)) {
        const float m_new = fmaxf(m_run, mx);
        const float alpha = m_new == -INFINITY ? 1.0f : fast_exp2(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int e = 0; e < 16; ++e) o[db][e] *= alpha;
        m_run = m_new;
      }
      const float m_use = m_run == -INFINITY ? 0.f : m_run;
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int v = 0; v < 16; ++v) s[v] = __builtin_fmaf(s[v], cc, -m_use);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int v = 0; v < 16; ++v) s[v] = fast_exp2(s[v]);
      __builtin_amdgcn_sched_barrier(0);
      float ps[2] = {0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        ps[i & 1] += s[2 * i] + s[2 * i + 1];
        pk[i] = pack_bf16x2(s[2 * i], s[2 * i + 1]);
      }
      l_run += ps[0] + ps[1];
      xp[w][0][lane] = u32x4_t{pk[0], pk[1], pk[2], pk[3]};
      xp[w][1][lane] = u32x4_t{pk[4], pk[5], pk[6], pk[7]};
    };

    // MFMA phase of step t: S(t) = Q K(t)^T over this wavefront's 32 keys (if QK), then O += P(t-1) V(t-1) over
    // its 128 dims (if PV); one slot per MFMA in a fixed order, each LDS operand read D = 4 MFMAs ahead. Then the
    // mask and row max of S(t), published for the partner.
    auto mfma_block = [&](auto pvc, auto qkc, const uint8_t* kb_t, const uint8_t* vb_prev) __attribute__((always_inline)) {
      constexpr bool PV = decltype(pvc)::value, QK = decltype(qkc)::value;
      constexpr int NQ = QK ? 16 : 0, NOPS = NQ + (PV ? 16 : 0), D = 4;
      bf16x8_t opr[D];
      bf16x8_t pp[2];  // the partner's P(t-1) fragments (k-steps 2 (1 - role) + j), read D slots before P.V
      // the K operand addresses are formed at each read from an opaque copy of the lane base (one XOR each, in
      // the matrix core's shadow) instead of being kept in 16 registers across the loop
      uint32_t kq = kbase;
      asm volatile("" : "+v"(kq));
      // operand i: i < NQ: K (k-step ks = i); then V^T (k-step ss = j / 4, dim block db = j % 4), j = i - NQ
      auto read = [&](auto ic) __attribute__((always_inline)) {
        constexpr int i = decltype(ic)::value;
        if constexpr (PV && i == NQ) {
          pp[0] = as_bf16x8(xp[partner][0][lane]);
          pp[1] = as_bf16x8(xp[partner][1][lane]);
        }
        if constexpr (i < NQ) {
          opr[i % D] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(kb_t + (kq ^ (32u * i))));
        } else {
          constexpr int j = i - NQ;
          opr[i % D] = v_operand<HD>(vb_prev, NDB * role + (j & 3), j >> 2, vbase);
        }
      };
      if constexpr (NOPS > 0) {
        static_for<0, D>([&](auto ic) __attribute__((always_inline)) { read(ic); });
        if constexpr (QK) {
#pragma unroll
          for (int e = 0; e < 16; ++e) s[e] = 0.f;
        }
        __builtin_amdgcn_sched_barrier(0);
        static_for<0, NOPS>([&](auto ic) __attribute__((always_inline)) {
          constexpr int i = decltype(ic)::value;
          if constexpr (i < NQ) {
            s = mfma32(opr[i % D], qf[i], s);
          } else {
            constexpr int j = i - NQ, ss = j >> 2, db = j & 3;
            // k-step ss covers keys 16 ss .. 16 ss + 15: this wavefront's own P when ss / 2 == role
            bf16x8_t pb;
            if ((ss >> 1) == role) {
              const int i0 = 4 * (ss & 1);
              pb = as_bf16x8(u32x4_t{pk[i0], pk[i0 + 1], pk[i0 + 2], pk[i0 + 3]});
            } else {
              pb = pp[ss & 1];
            }
            o[db] = mfma32(opr[i % D], pb, o[db]);
          }
          if constexpr (i + D < NOPS) read(std::integral_constant<int, i + D>{});
          __builtin_amdgcn_sched_barrier(0);
        });
      }
    };
    auto mfma_phase = [&](int t, const uint8_t* kb_t, const uint8_t* vb_prev) __attribute__((always_inline)) {
      const bool pv = t >= 1 && (t - 1) * T::BN <= wmax;
      const bool qk = t < t_end && t * T::BN <= wmax;
      using Y = std::true_type;
      using N = std::false_type;
      // the MFMA phase at a raised wave priority: where the SIMD's two wavefronts compete for an issue slot, the
      // one feeding the matrix core goes first, ahead of its partner's softmax and tile loads (config 5: 9.03 ->
      // 8.74 ms, same box, alternated; the head_dim-128 kernel, whose loads go out from its MFMA phase, gains
      // nothing from it)
      __builtin_amdgcn_s_setprio(1);
      if (pv && qk)
        mfma_block(Y{}, Y{}, kb_t, vb_prev);
      else if (pv)
        mfma_block(Y{}, N{}, kb_t, vb_prev);
      else if (qk)
        mfma_block(N{}, Y{}, kb_t, vb_prev);
      __builtin_amdgcn_s_setprio(0);
      if (qk) {
        const int k0 = t * T::BN + 32 * role;
        if (k0 + 31 > wmin) {  // the keys straddle some row's last visible key
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int key = k0 + 8 * (v >> 2) + 4 * hf + (v & 3);
            if (key > lim) s[v] = -INFINITY;
          }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[v]);
        m_own = halves_max(mx) * cc;
        if (hf == 0) xm[w][lr] = m_own;
      }
    };
    // Tile loads (group 1 only): the 32 direct-to-LDS loads of a 64-key x 256-dim tile, 8 per wavefront of the
    // group. Load c = 8 gu + i writes bytes [1024 c, 1024 c + 1024) of the tile: lane l lands on row
    // r = 16 gu + 2 i + l / 32, swizzled unit l % 32, so it fetches the logical unit u = (l % 32) ^ swz(r). With
    // r & 3 = (2i & 3) | hf and (r >> 2) & 3 = (i >> 1) & 3, swz(r) = c_i | (hf << 2), c_i = ((2i & 3) << 2) |
    // ((i >> 1) & 3): the byte offset in a whole tile is (16 gu + hf) 2 stride + 4 i stride + 16 ((l % 32) ^
    // (hf << 2) ^ c_i), a per-lane base plus a per-load constant, so no per-load offsets stay in registers.
    const uint32_t lu16 = (uint32_t)(((lane & 31) ^ (hf << 2)) << 4);
    auto tile_load = [&](uint8_t* buf, const uint16_t* base, long long stride, bool fast, int k0) __attribute__((always_inline)) {
      const uint32_t m0b = (uint32_t)reinterpret_cast<uintptr_t>(buf) + gu * 8 * 1024;
      if (fast && k0 + T::BN <= Nb) {
        const uint8_t* tb = reinterpret_cast<const uint8_t*>(base + (long long)k0 * stride);
        uint32_t lb = (uint32_t)((16 * (int)gu + hf) * 2 * stride);
        asm volatile("" : "+v"(lb));
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t ci = (uint32_t)((((2 * i) & 3) << 2) | ((i >> 1) & 3));
          const uint32_t off = lb + (uint32_t)(4 * i * stride) + (lu16 ^ (ci << 4));
          asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(tb + off), "{m0}"(m0b + i * 1024) : "memory");
        }
      } else {
        // a partial last tile: rows beyond the window's last key read that key (their scores are masked)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          int rr, uu, ln = lane;
          asm volatile("" : "+v"(ln));
          Dma<HD, 4>::slot((int)gu, i, ln, rr, uu);
          const int key = min(k0 + rr, Nb - 1);
          asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(base + (long long)key * stride + 8 * uu),
                       "{m0}"(m0b + i * 1024) : "memory");
        }
      }
    };
    // the loads of step t, split over both halves so that the memory pipeline streams through the whole step:
    // K(t+1) by group 1 at the start of half 1, V(t) by group 0 at the start of half 2, each before its group's
    // softmax; both land before the end-of-step barrier
    auto load_k = [&](int t) __attribute__((always_inline)) {
      if (t + 1 < t_end) tile_load(kring[(t + 1) & 1], Kb, p.ksM, kfast, (t + 1) * T::BN);
    };
    auto load_v = [&](int t) __attribute__((always_inline)) {
      if (t < t_end) tile_load(vring[t & 1], Vb, p.vsM, vfast, t * T::BN);
    };

    if (t_end > 0) {
      if (grp == 1) tile_load(kring[0], Kb, p.ksM, kfast, 0);
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      __syncthreads();
      for (int t = 0; t <= t_end; ++t) {
        const uint8_t* kb_t = kring[t & 1];
        const uint8_t* vb_prev = vring[(t + 1) & 1];
        if (grp == 0) {
          mfma_phase(t, kb_t, vb_prev);
        } else {
          load_k(t);  // before the softmax: ~0.7% faster on config 5 than after it (the loads get longer to land)
          if (t >= 1) softmax(t - 1);
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wavefront's xm / xp writes are visible ...
        exec_barrier();                      // ... to its partner after the barrier (the tile loads stay in flight)
        if (grp == 0) {
          load_v(t);
          if (t < t_end) softmax(t);
        } else {
          mfma_phase(t, kb_t, vb_prev);
        }
        // K(t+1) and V(t), issued in this step, must have landed (vmcnt(0)); every wavefront is done with K(t)
        // and V(t-1), which the next step's loads replace
        __builtin_amdgcn_s_waitcnt(0x0F70);
        __syncthreads();
      }
    }

    // ---- epilogue: the pair's row sums meet in LDS; normalise, LSE, store this wavefront's 128 dims
    const float l_own = halves_sum(l_run);  // a cross-half lane swap: every lane must be active here
    if (hf == 0) xl[w][lr] = l_own;
    __syncthreads();
    const float l = xl[w][lr] + xl[partner][lr];  // the same sum in both wavefronts of the pair
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    if (!rvalid) return;
    if (p.lse && hf == 0 && role == 0) {
      const float lse = l > 0.f ? (m_run + log2f(l)) * 0.69314718055994530942f : -INFINITY;
      p.lse[(long long)b * p.lsB + (long long)hk * p.lsH + (tok0 + tok) * p.lsT + (long long)g * p.lsG] = lse;
    }
    if (POST) {
      // attn_post (v11:451-522): token row R = inv[b*Lq + tok], query head hk*G + g; R < 0 rows are padding
      const int R = p.inv[(long long)b * p.Lq + tok];
      if (R < 0) return;
      const long long hq = (long long)hk * p.G + g;
      const uint16_t* grow = p.qg + (long long)R * p.qg_rs + hq * (2 * HD) + HD;
      uint16_t* orow = p.outp + (long long)R * p.out_rs + hq * HD;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int d = 32 * (NDB * role + db) + 8 * q4 + 4 * hf;
          const u32x2_t gw = *reinterpret_cast<const u32x2_t*>(grow + d);
          const uint32_t ob0 = pack_bf16x2(o[db][4 * q4 + 0] * inv, o[db][4 * q4 + 1] * inv);
          const uint32_t ob1 = pack_bf16x2(o[db][4 * q4 + 2] * inv, o[db][4 * q4 + 3] * inv);
          const uint32_t s0 = sigmoid_bf16_bits(gw[0] & 0xffffu), s1 = sigmoid_bf16_bits(gw[0] >> 16);
          const uint32_t s2 = sigmoid_bf16_bits(gw[1] & 0xffffu), s3 = sigmoid_bf16_bits(gw[1] >> 16);
          u32x2_t res;
          res[0] = pack_bf16x2(bf16lo(ob0) * bf16lo(s0), bf16hi(ob0) * bf16lo(s1));
          res[1] = pack_bf16x2(bf16lo(ob1) * bf16lo(s2), bf16hi(ob1) * bf16lo(s3));
          *reinterpret_cast<u32x2_t*>(orow + d) = res;
        }
      return;
    }
    if (!p.o) return;
    uint16_t* orow = p.o + (long long)b * p.osB + (long long)hk * p.osH + (tok0 + tok) * p.osT + (long long)g * p.osG;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d = 32 * (NDB * role + db) + 8 * q4 + 4 * hf;
        const uint32_t w0 = pack_bf16x2(o[db][4 * q4 + 0] * inv, o[db][4 * q4 + 1] * inv);
        const uint32_t w1 = pack_bf16x2(o[db][4 * q4 + 2] * inv, o[db][4 * q4 + 3] * inv);
        if (o_vec8) {
          *reinterpret_cast<u32x2_t*>(orow + d) = u32x2_t{w0, w1};
        } else {
          *reinterpret_cast<uint32_t*>(orow + d) = w0;
          *reinterpret_cast<uint32_t*>(orow + d + 2) = w1;
        }
      }
  };  // item

  const int P = gridDim.x;
  for (int it = 0;; ++it) {
    long long vid;
    if (xcd_aware) {
      const int x = blockIdx.x & 7, m = blockIdx.x >> 3, PX = P >> 3;
      vid = 8ll * ((long long)it * PX + ((it & 1) ? PX - 1 - m : m)) + x;
    } else {
      vid = (long long)it * P + ((it & 1) ? P - 1 - (int)blockIdx.x : (int)blockIdx.x);
    }
    if (vid >= n_items) break;
    // every wavefront is done with the previous item's LDS (its last reads were followed by a full barrier); not
    // __syncthreads(): its fence would wait for the previous item's output stores
    exec_barrier();
    item((int)vid);
  }
}

template <int MODE, bool POST>
static int launch_t(FwdParams p, hipStream_t stream) {
  p.n_tiles = (int)(((long long)p.M + PR_BM - 1) / PR_BM);
  const long long n_items = (long long)p.B * p.H * p.n_tiles;
  // an empty grid is rejected before any HIP call, as the reference's zero-sized launch would fail
  if (n_items <= 0 || n_items > INT_MAX) return (int)hipErrorInvalidConfiguration;
  const int cus = device_cus(stream);
  if (cus <= 0) return (int)hipErrorInvalidDevice;
  const long long nwg = n_items < cus ? n_items : cus;  // one workgroup per CU (its LDS and registers fill one)
  const int o_vec8 = (!POST && p.o) ? (aligned_elems(p.o, 4, {p.osB, p.osH, p.osT, p.osG}) ? 1 : 0) : 0;
  hipLaunchKernelGGL((fmha_fwd_pair_kernel<MODE, POST>), dim3((unsigned)nwg), dim3(64 * PR_NW), 0, stream, p, o_vec8);
  return (int)hipGetLastError();
}

int launch_fwd_pair(const FwdParams& p, int mode, bool post, hipStream_t stream) {
  if (mode == MODE_QPOS) return post ? launch_t<MODE_QPOS, true>(p, stream) : launch_t<MODE_QPOS, false>(p, stream);
  if (mode == MODE_VARLEN && !post) return launch_t<MODE_VARLEN, false>(p, stream);
  return (int)hipErrorInvalidValue;
}

}  // namespace reax
