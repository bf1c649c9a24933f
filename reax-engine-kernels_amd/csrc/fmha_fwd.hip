// FA2-style attention forward for gfx950 (CDNA4), the MI355X rebuild of the REAX FMHA path:
//   reference: libreax_howu/reax_fmha_v8.cu (fmha3_kernel, launch2) and libreax_fmha_post/reax_fmha_v11.cu
//   (the same kernel with the POST gate epilogue).
//
// Design (one workgroup = 4 wavefronts = 128 folded query rows of one (batch, KV head)):
//   - A lane owns one query row: S^T = K . Q^T is computed with v_mfma_f32_32x32x16_bf16 where the A operand is
//     a K fragment (32 keys x 16 dims, read from LDS) and the B operand is the lane's Q row fragment (kept in
//     registers for the whole key loop). The 32x32 accumulator layout then gives lane l the scores of query
//     l%32 for 16 keys, so the row max / row sum need only in-lane work plus one permlane32 swap.
//   - The same registers, converted to bf16, are the B operand of O^T = V^T . P^T: no data movement between
//     the two MFMA stages. The key order inside each 16-key MFMA step follows the accumulator layout, and the
//     V^T operand is read in that order from the row-major V tile with ds_read_b64_tr_b16 (gfx950's transposing
//     LDS read).
//   - K/V tiles of 64 keys stream straight from HBM into LDS (global_load_lds_dwordx4), double-buffered, one
//     barrier per tile; the S^T of the next tile is computed before the softmax of the current one. Rows use a
//     16-byte-unit XOR swizzle that keeps both the K operand reads and the transposed V reads bank-conflict free.
//   - Online softmax in base 2 on v_exp_f32 with the running max in log2 units; the O rescale runs only when a
//     row max grows by more than 2^8 (probabilities stay <= 2^8).
//   - Causal / qpos tiles visit only key tiles that some row of the workgroup can see (v8:155-162, 237); the
//     per-element mask is applied only to tiles that straddle a row's limit. Workgroups are dispatched heaviest
//     first (v8:134-135) and, when B*H is a multiple of 8, each XCD's L2 serves a fixed set of KV heads.
#include "fmha_common.h"
#include "fmha_launch.h"
#include "fmha_sched.h"
#include "fmha_tiles.h"

#include <atomic>
#include <climits>
#include <type_traits>

namespace reax {


template <int HD, int MODE, bool POST, bool SPLIT>
__global__ void __launch_bounds__(256, HD == 128 ? 2 : 1) fmha_fwd_kernel(const FwdParams p, int o_vec8) {
  using T = FwdTile<HD>;
  __shared__ __align__(1024) uint8_t kbuf0[T::TILE];
  __shared__ __align__(1024) uint8_t kbuf1[T::TILE];
  __shared__ __align__(1024) uint8_t vbuf0[T::TILE];
  __shared__ __align__(1024) uint8_t vbuf1[T::TILE];
  __shared__ int s_lim[4];
  __shared__ int s_raw[4];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, hf = lane >> 5, lr = lane & 31;

  // ---- workgroup -> (batch, KV head, row tile[, key split]): heaviest tile first; when B*H % 8 == 0 each
  // XCD (workgroups are dealt to the 8 XCDs round-robin) serves a fixed set of KV heads from its own L2
  const int BH = p.B * p.H;
  int id = blockIdx.x, split = 0;
  if (SPLIT) {
    split = id % p.num_splits;
    id /= p.num_splits;
  }
  int bh, rank;
  if (!SPLIT && (BH & 7) == 0) {
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
  const int r0 = tile * T::BM;
  if (r0 >= Mb) return;  // uniform over the workgroup (ragged varlen tail)

  // ---- this lane's query row and its last visible key
  const int r = r0 + 32 * w + lr;
  const bool rvalid = r < Mb;
  const int tok = rvalid ? r / p.G : 0;
  const int g = rvalid ? r - tok * p.G : 0;
  int lim = -1, qraw = -1;
  if (rvalid) {
    if (MODE == MODE_QPOS) {
      qraw = p.qpos[(long long)b * p.qpBs + tok];
      lim = min(qraw, Nb - 1);
    } else if (MODE == MODE_VARLEN) {
      lim = min(tok, Nb - 1);
    } else {
      lim = Nb - 1;
    }
    lim = max(lim, -1);
  }
  // key window of this workgroup: [kbeg, kend); split_len is a multiple of the tile size
  int kbeg = 0, kend = Nb;
  if (SPLIT) {
    kbeg = split * p.split_len;
    kend = min(Nb, kbeg + p.split_len);
    lim = min(lim, kend - 1);
    if (lim < kbeg) lim = -1;
  }
  const bool blk0 = MODE == MODE_QPOS && !SPLIT && p.qpos0_block;
  int wmax = wave_max(lim), wmin = wave_min(lim);
  if (blk0) {
    // the reference's 64-row blocks start at multiples of 64, so with 128-row tiles wavefronts 2j and 2j + 1 (32
    // rows each) make up one block: when the block's largest raw qpos is 0, every live row of it sees key 0 only,
    // which stores V[0] (the raw value: a row with qpos > N - 1 = 0 does not trigger the shortcut)
    const int rmax = wave_max(qraw);
    if (lane == 0) s_raw[w] = rmax;
  }
  if (lane == 0) s_lim[w] = wmax;
  __syncthreads();
  if (blk0) {
    const int bmax = max(s_raw[w & ~1], s_raw[w | 1]);
    if (bmax == 0 && rvalid && Nb > 0) lim = 0;
    wmax = wave_max(lim);
    wmin = wave_min(lim);
  }
  const int cmax = max(max(s_lim[0], s_lim[1]), max(s_lim[2], s_lim[3]));
  const int t_beg = kbeg / T::BN;
  const int t_end = cmax < kbeg ? t_beg : cmax / T::BN + 1;  // key tiles [t_beg, t_end)

  // ---- Q fragments: B operand of S^T = K Q^T (dims 16*ks + 8*hf .. +7 of this lane's row)
  const uint16_t* qrow = p.q + (long long)b * p.qsB + (long long)hk * p.qsH + (tok0 + tok) * p.qsT + (long long)g * p.qsG;
  bf16x8_t qf[T::QK];
#pragma unroll
  for (int ks = 0; ks < T::QK; ++ks)
    qf[ks] = as_bf16x8(rvalid ? ld16(qrow + 16 * ks + 8 * hf) : u32x4_t{0u, 0u, 0u, 0u});

  const uint16_t* Kb = p.k + (long long)b * p.ksB + (long long)hk * p.ksH + tok0 * p.ksM;
  const uint16_t* Vb = p.v + (long long)b * p.vsB + (long long)hk * p.vsH + tok0 * p.vsM;

  f32x16_t o[T::DB];
#pragma unroll
  for (int db = 0; db < T::DB; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[db][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  // BIAS mode turns the scores into log2-domain logits in place, so its exponent multiplier is 1
  const float cc = MODE == MODE_BIAS ? 1.0f : p.scale_log2;
  const uint16_t* brow = nullptr;
  if (MODE == MODE_BIAS)
    brow = p.bias + (long long)b * p.bsB + (long long)hk * p.bsH + (long long)(rvalid ? r : 0) * p.bsM;

  // ---- pipeline: iteration t reads K(t+1) and V(t) while K(t+2) and V(t+1) stream into the other buffers
  const Dma<HD, 4> kplan(p.ksM, w, lane), vplan(p.vsM, w, lane);
  const bool kfast = p.ksM * 2 * T::BN < (1ll << 31), vfast = p.vsM * 2 * T::BN < (1ll << 31);
  const uint32_t kbase[2] = {k_lane_base<HD>(0, lr, hf), k_lane_base<HD>(1, lr, hf)};
  const uint32_t vbase = v_lane_base<HD>(lane);
  f32x16_t sa[2];
  if (t_end > t_beg) {
    kplan.tile(kbuf0, Kb, p.ksM, kfast, t_beg * T::BN, kend, w, lane);
    vplan.tile(vbuf0, Vb, p.vsM, vfast, t_beg * T::BN, kend, w, lane);
    if (t_beg + 1 < t_end) kplan.tile(kbuf1, Kb, p.ksM, kfast, (t_beg + 1) * T::BN, kend, w, lane);
    wait_dma_and_sync();
    if (t_beg * T::BN <= wmax) qk_tile<HD>(sa, kbuf0, qf, kbase);
    __syncthreads();  // kbuf0 is refilled in the first iteration
  }

  // One pipeline step on tile t: s_cur holds S(t), s_nxt receives S(t+1); kb_next holds K(t+1), vb_cur V(t),
  // while kb_fill / vb_fill receive K(t+2) / V(t+1). The loop below is unrolled by two so the score buffers and
  // LDS buffers swap roles at compile time (no register copies, constant LDS addresses).
  auto step = [&](int t, f32x16_t(&s_cur)[2], f32x16_t(&s_nxt)[2], const uint8_t* kb_next, uint8_t* kb_fill,
                  const uint8_t* vb_cur, uint8_t* vb_fill) {
    const int k0 = t * T::BN;
    if (t + 2 < t_end) kplan.tile(kb_fill, Kb, p.ksM, kfast, k0 + 2 * T::BN, kend, w, lane);
    if (t + 1 < t_end) vplan.tile(vb_fill, Vb, p.vsM, vfast, k0 + T::BN, kend, w, lane);
    const bool nxt = t + 1 < t_end && k0 + T::BN <= wmax;
    if (k0 <= wmax) {
      if (MODE == MODE_BIAS) {
        // x = (s*scale + bias) * log2(e), bias read only for keys inside the sequence (v8:279-280)
        const float l2e = 1.44269504088896340736f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int key = k0 + 32 * kb + 8 * (v >> 2) + 4 * hf + (v & 3);
            const float bv = (rvalid && key < Nb) ? __uint_as_float((uint32_t)brow[key] << 16) : 0.f;
            s_cur[kb][v] = (s_cur[kb][v] * p.scale + bv) * l2e;
          }
      }
      if (k0 + T::BN - 1 > wmin) {  // the tile straddles some row's last visible key
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int key = k0 + 32 * kb + 8 * (v >> 2) + 4 * hf + (v & 3);
            if (key > lim) s_cur[kb][v] = -INFINITY;
          }
      }
      // ---- online softmax (log2 domain) with lazy rescaling
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s_cur[kb][v]);
      mx = halves_max(mx) * cc;
      if (__any(mx > m_run + RESCALE_SLACK)) {
        const float m_new = fmaxf(m_run, mx);
        const float alpha = m_new == -INFINITY ? 1.0f : fast_exp2(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < T::DB; ++db)
#pragma unroll
          for (int e = 0; e < 16; ++e) o[db][e] *= alpha;
        m_run = m_new;
      }
      const float m_use = m_run == -INFINITY ? 0.f : m_run;
      // straight-line block: S(t+1) MFMAs interleaved with the exponentials of tile t, then O += V(t)^T P^T
      auto body = [&](auto with_next) __attribute__((always_inline)) {
        constexpr bool NEXT = decltype(with_next)::value;
        float psum = 0.f;
        uint32_t pk[2][8];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float p0 = fast_exp2(__builtin_fmaf(s_cur[kb][2 * i], cc, -m_use));
            const float p1 = fast_exp2(__builtin_fmaf(s_cur[kb][2 * i + 1], cc, -m_use));
            psum += p0;
            psum += p1;
            pk[kb][i] = pack_bf16x2(p0, p1);
          }
        l_run += psum;
#pragma unroll
        for (int ss = 0; ss < 4; ++ss) {
          const u32x4_t pw = {pk[ss >> 1][4 * (ss & 1) + 0], pk[ss >> 1][4 * (ss & 1) + 1],
                              pk[ss >> 1][4 * (ss & 1) + 2], pk[ss >> 1][4 * (ss & 1) + 3]};
          const bf16x8_t pb = as_bf16x8(pw);
#pragma unroll
          for (int db = 0; db < T::DB; ++db) o[db] = mfma32(v_operand<HD>(vb_cur, db, ss, vbase), pb, o[db]);
        }
        if (NEXT) {
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int e = 0; e < 16; ++e) s_nxt[kb][e] = 0.f;
#pragma unroll
          for (int ks = 0; ks < T::QK; ++ks)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
              const u32x4_t kf = *reinterpret_cast<const u32x4_t*>(kb_next + (kbase[kb] ^ (32u * ks)));
              s_nxt[kb] = mfma32(as_bf16x8(kf), qf[ks], s_nxt[kb]);
            }
        }
      };
      if (nxt)
        body(std::integral_constant<bool, true>{});
      else
        body(std::integral_constant<bool, false>{});
    } else if (nxt) {
      qk_tile<HD>(s_nxt, kb_next, qf, kbase);
    }
    wait_dma_and_sync();
  };

  for (int t = t_beg; t < t_end; t += 2) {
    step(t, sa, sa, kbuf1, kbuf0, vbuf0, vbuf1);
    if (t + 1 < t_end) step(t + 1, sa, sa, kbuf0, kbuf1, vbuf1, vbuf0);
  }

  // ---- epilogue: normalise, LSE, store (O^T layout: lane holds dims 32db + 8(v/4) + 4hf + v%4 of its row)
  const float l = halves_sum(l_run);
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  if (!rvalid) return;
  if (SPLIT) {
    // partial result of this key split: O / l (fp32) and its LSE (natural log), -inf when nothing is visible
    const long long prow = ((long long)bh * p.num_splits + split) * p.M + r;
    if (hf == 0) p.ws_lse[prow] = l > 0.f ? (m_run + log2f(l)) * 0.69314718055994530942f : -INFINITY;
    float* po = p.ws_o + prow * HD;
#pragma unroll
    for (int db = 0; db < T::DB; ++db)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d = 32 * db + 8 * q4 + 4 * hf;
        *reinterpret_cast<f32x4_t*>(po + d) =
            f32x4_t{o[db][4 * q4 + 0] * inv, o[db][4 * q4 + 1] * inv, o[db][4 * q4 + 2] * inv, o[db][4 * q4 + 3] * inv};
      }
    return;
  }
  if (p.lse && hf == 0) {
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
    for (int db = 0; db < T::DB; ++db)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int d = 32 * db + 8 * q4 + 4 * hf;
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
  for (int db = 0; db < T::DB; ++db)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = 32 * db + 8 * q4 + 4 * hf;
      const uint32_t w0 = pack_bf16x2(o[db][4 * q4 + 0] * inv, o[db][4 * q4 + 1] * inv);
      const uint32_t w1 = pack_bf16x2(o[db][4 * q4 + 2] * inv, o[db][4 * q4 + 3] * inv);
      if (o_vec8) {
        *reinterpret_cast<u32x2_t*>(orow + d) = u32x2_t{w0, w1};
      } else {
        *reinterpret_cast<uint32_t*>(orow + d) = w0;
        *reinterpret_cast<uint32_t*>(orow + d + 2) = w1;
      }
    }
}

// ------------------------------------------------------------------------------------------------------------
// Ping-pong forward for head_dim 128 (qpos / varlen, O + LSE): 8 wavefronts = 256 folded rows per workgroup.
// Wavefronts w and w + 4 run on the same SIMD (the dispatcher deals a workgroup's wavefronts round-robin over the
// CU's 4 SIMDs), so the workgroup is split into group 0 (w < 4, rows 0..127) and group 1 (w >= 4, rows
// 128..255) that alternate phases at every half-step barrier:
//     half 1 of step t: group 0 runs its MFMA phase  [P(t-1).V(t-1), then S(t) = K(t).Q^T]
//                       group 1 runs its VALU phase  [softmax of S(t-1) -> P(t-1)]
//     half 2 of step t: the roles swap.
// While one wavefront of a SIMD keeps the matrix core busy, the other one does its exponentials, so the
// MFMA pipe never waits for a softmax. K(t+1) and V(t) stream into LDS during step t (two buffers each): group 0
// issues all of a step's loads, one after every fourth MFMA of its MFMA phase (measured: the 32 direct-to-LDS
// loads of a step issued by all wavefronts at the start of the step held each of them up for ~480 clocks; spread
// this way they cost group 0 ~45 clocks each, while its matrix core work continues).
// Q and O cross between HBM and registers through LDS (8 KB per wavefront): the loads and stores of 32 rows
// spread over 32 rows each (16 bytes per row per instruction) kept an item's prologue and epilogue at ~4 us each;
// as 1 KB copies of four whole rows they are ~4% of config 2 faster. The Q copies and the first K tile go out
// before the row limits are worked out.
constexpr int PP_NW = 8;
constexpr int PP_STAGES = 2;
constexpr int PP_BM = 256;

template <int MODE, int NS>
__global__ void __launch_bounds__(512, 1) fmha_fwd_pp_kernel(const FwdParams p, int o_vec) {
  constexpr int HD = 128;
  using T = FwdTile<HD>;
  static_assert(NS == 2, "two K/V stages: K(0) is the only tile the prologue loads, with Q");
  // one block, the K/V ring first: its operand reads reach every stage with an instruction's 16-bit offset.
  // qo: each wavefront's 32 rows, Q on the way in and O on the way out (row-major, 16-byte units swizzled by
  // swz(row)), so that both move between HBM and LDS as whole rows, four per 1 KB copy
  struct Lds {
    uint8_t kring[NS][T::TILE];
    uint8_t vring[NS][T::TILE];
    uint8_t qo[PP_NW][32 * HD * 2];
  };
  __shared__ __align__(1024) Lds L;
  auto& kring = L.kring;
  auto& vring = L.vring;
  auto& qo = L.qo;
  __shared__ int s_lim[PP_NW];
  __shared__ std::conditional_t<MODE == MODE_VARLEN, VarlenSched, char> vs;  // varlen item schedule
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, hf = lane >> 5, lr = lane & 31;
  const int grp = w >> 2;
  const uint32_t wu = __builtin_amdgcn_readfirstlane(w);  // the wavefront index as a scalar, for load addresses

  // ---- persistent workgroups: the grid has at most one workgroup per CU, and each works through items (row
  // tiles of one (batch, KV head)) in a fixed order. Item ids follow the work order, heaviest tile first; when
  // B*H % 8 == 0 the 8 XCDs (workgroups are dealt to them round-robin) each own the KV heads bh = x mod 8, so
  // a head's K/V stays in one XCD's L2 (not for varlen, whose sequences differ in length: there a fixed
  // head-to-XCD split leaves some XCDs with more work than others). Within its class, workgroup m takes items m, 2P'-1-m, 2P'+m, ... (P'
  // workgroups in the class): a heavy item and a light one in turn, so the per-workgroup work evens out without
  // relying on the order in which the hardware hands workgroups to CUs.
  const int BH = p.B * p.H;
  const long long n_items = (long long)BH * p.n_tiles;
  const bool xcd_aware = MODE != MODE_VARLEN && (BH & 7) == 0 && (gridDim.x & 7) == 0;
  // item (bh, tile): row tile `tile` of (batch or sequence bh / H, KV head bh % H). with_rounds (varlen only): the
  // schedule's rounds run in wavefront 0 while this item's first loads are in flight, before its first barrier
  auto item = [&](int bh, int tile, bool with_rounds) __attribute__((always_inline)) {
  const int b = bh / p.H, hk = bh - b * p.H;
  long long tok0 = 0;
  int Mb = p.M, Nb = p.N;
  if (MODE == MODE_VARLEN) {
    const int s0 = p.cu_seqlens[b], s1 = p.cu_seqlens[b + 1];
    tok0 = s0;
    Nb = s1 - s0;
    Mb = Nb * p.G;
  }
  const int r0 = tile * PP_BM;
  if (r0 >= Mb) {  // uniform over the workgroup
    if constexpr (MODE == MODE_VARLEN) {
      if (with_rounds) {
        vs_rounds(vs, gridDim.x, blockIdx.x);
        __syncthreads();
      }
    }
    return;
  }

  const int r = r0 + 32 * w + lr;
  const bool rvalid = r < Mb;
  const int tok = rvalid ? r / p.G : 0;
  const int g = rvalid ? r - tok * p.G : 0;
  bf16x8_t qf[T::QK];
  const uint16_t* Kb = p.k + (long long)b * p.ksB + (long long)hk * p.ksH + tok0 * p.ksM;
  const uint16_t* Vb = p.v + (long long)b * p.vsB + (long long)hk * p.vsH + tok0 * p.vsM;
  const uint16_t* qb = p.q + (long long)b * p.qsB + (long long)hk * p.qsH + tok0 * p.qsT;
  {
    // load i: lane l fetches row lrow = 4i + l/16 of the wavefront's 32 (token tq, head gq; rows past the tile's
    // end read its last row), logical unit (l % 16) ^ swz(lrow)
    const int lrow0 = lane >> 4, pu = lane & 15;
    const int row0 = r0 + 32 * w + lrow0;
    int tq = row0 / p.G, gq = row0 - tq * p.G;
    const int d4 = 4 / p.G, m4 = 4 - d4 * p.G;
    const int ltok = (Mb - 1) / p.G, lg = Mb - 1 - ltok * p.G;
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)reinterpret_cast<uintptr_t>(&qo[w][0]));
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = r0 + 32 * w + 4 * i + lrow0;
      const bool ok = row < Mb;
      const int u = pu ^ swz(4 * i + lrow0);
      const uint16_t* src = qb + (long long)(ok ? tq : ltok) * p.qsT + (long long)(ok ? gq : lg) * p.qsG + 8 * u;
      asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(m0 + i * 1024) : "memory");
      tq += d4;
      gq += m4;
      if (gq >= p.G) { gq -= p.G; ++tq; }
    }
  }
  const Dma<HD, PP_NW / 2> kplan(p.ksM, w, lane), vplan(p.vsM, w, lane);  // used by group 0 only
  const bool kfast = p.ksM * 2 * T::BN < (1ll << 31), vfast = p.vsM * 2 * T::BN < (1ll << 31);
  // the first K tile goes out with Q (an item whose rows see no key only wastes it)
  if (grp == 0 && Nb > 0) {
    int ln = lane;
    asm volatile("" : "+v"(ln));  // per-lane terms formed here, not hoisted out of the item loop
    kplan.template tile<1>(kring[0], Kb, p.ksM, kfast, 0, Nb, (int)wu, ln);
  }
  int lim = -1;
  if (rvalid) {
    lim = MODE == MODE_QPOS ? min(p.qpos[(long long)b * p.qpBs + tok], Nb - 1) : min(tok, Nb - 1);
    lim = max(lim, -1);
  }
  // wmin: the smallest limit among the wavefront's rows inside the tile. Rows past its end are never stored, so
  // they must not force the mask pass onto every key tile of a partial row tile.
  const int wmax = wave_max(lim), wmin = wave_min(rvalid ? lim : INT_MAX);
  if (lane == 0) s_lim[w] = wmax;
  if constexpr (MODE == MODE_VARLEN) {
    if (with_rounds) vs_rounds(vs, gridDim.x, blockIdx.x);  // the barrier below orders S.mine[] before its reads
  }
  // the Q and K(0) copies are inline assembly, which the compiler does not count: wait for them explicitly
  // (the barrier's own fence only drains the loads it knows of)
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __syncthreads();
  int cmax = s_lim[0];
#pragma unroll
  for (int i = 1; i < PP_NW; ++i) cmax = max(cmax, s_lim[i]);
  const int t_end = cmax < 0 ? 0 : cmax / T::BN + 1;
  // the wait and barrier above: this wavefront's Q copies and group 0's K(0) copies have landed
  {
    int ln = lane;
    asm volatile("" : "+v"(ln));  // addresses formed here, not kept live from the kernel's start
    const uint32_t qa = (uint32_t)reinterpret_cast<uintptr_t>(&qo[w][0]) + k_lane_base<HD>(0, ln & 31, ln >> 5);
#pragma unroll
    for (int ks = 0; ks < T::QK; ++ks)
      qf[ks] = as_bf16x8(*reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(qa ^ (32u * ks)));
  }


  f32x16_t o[T::DB];
#pragma unroll
  for (int db = 0; db < T::DB; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[db][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const float cc = p.scale_log2;
  f32x16_t s[2];
  uint32_t pk[2][8];

  const uint32_t kbase[2] = {k_lane_base<HD>(0, lr, hf), k_lane_base<HD>(1, lr, hf)};
  const uint32_t vbase = v_lane_base<HD>(lane);

  // softmax of tile t: S in s[] -> P in pk[] (bf16), running max / row sum, lazy O rescale
  // softmax_core<MASK>: MASK = false only where the caller knows that every row of the wavefront sees the whole tile
  auto softmax_core = [&](auto maskc, int k0) __attribute__((always_inline)) {
    if (decltype(maskc)::value && k0 + T::BN - 1 > wmin) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = k0 + 32 * kb + 8 * (v >> 2) + 4 * hf + (v & 3);
          if (key > lim) s[kb][v] = -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[kb][v]);
    mx = halves_max(mx) * cc;
    if (__any(mx > m_run + RESCALE_SLACK)) {
      const float m_new = fmaxf(m_run, mx);
      const float alpha = m_new == -INFINITY ? 1.0f : fast_exp2(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < T::DB; ++db)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[db][e] *= alpha;
      m_run = m_new;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    // three passes over the 32 elements (arguments, exponentials, sums and packing) with scheduling barriers in
    // between: every instruction of a pass is independent of the others, so one wavefront issues them back to
    // back instead of waiting on each exponential's input and result in turn
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) s[kb][v] = __builtin_fmaf(s[kb][v], cc, -m_use);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) s[kb][v] = fast_exp2(s[kb][v]);
    __builtin_amdgcn_sched_barrier(0);
    float ps[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        ps[(i & 1) * 2] += s[kb][2 * i];
        ps[(i & 1) * 2 + 1] += s[kb][2 * i + 1];
        pk[kb][i] = pack_bf16x2(s[kb][2 * i], s[kb][2 * i + 1]);
      }
    l_run += (ps[0] + ps[1]) + (ps[2] + ps[3]);
  };
  auto softmax = [&](int t) __attribute__((always_inline)) {
    const int k0 = t * T::BN;
    if (k0 > wmax) return;
    softmax_core(std::true_type{}, k0);
  };
  // MFMA phase of step t: O += V(t-1)^T P(t-1)^T (if PV), then S(t) = K(t) Q^T (if QK), one slot per MFMA in a
  // fixed order (scheduling barriers between slots): each LDS operand read goes out D = 4 MFMAs ahead of its
  // use, and dma(j), j = 0..7, one of the step's tile loads, after every (NOPS / 8)-th MFMA.
  auto mfma_block = [&](auto pvc, auto qkc, const uint8_t* kb_t, const uint8_t* vb_prev,
                        auto&& dma) __attribute__((always_inline)) {
    constexpr bool PV = decltype(pvc)::value, QK = decltype(qkc)::value;
    constexpr int NP = PV ? 16 : 0, NOPS = NP + (QK ? 16 : 0), D = 4;
    bf16x8_t opr[D];
    // operand i: i < NP: V^T (k-step ss = i/4, dim block db = i%4); then K (kb = j%2, ks = j/2), j = i - NP
    auto read = [&](auto ic) __attribute__((always_inline)) {
      constexpr int i = decltype(ic)::value;
      if constexpr (i < NP) {
        opr[i % D] = v_operand<HD>(vb_prev, i & 3, i >> 2, vbase);
      } else {
        constexpr int j = i - NP;
        opr[i % D] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(kb_t + (kbase[j & 1] ^ (32u * (j >> 1)))));
      }
    };
    if constexpr (NOPS == 0) {
      static_for<0, 8>([&](auto jc) __attribute__((always_inline)) { dma(decltype(jc)::value); });
    } else {
      static_for<0, D>([&](auto ic) __attribute__((always_inline)) { read(ic); });
      if constexpr (QK) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int e = 0; e < 16; ++e) s[kb][e] = 0.f;
      }
      __builtin_amdgcn_sched_barrier(0);
      static_for<0, NOPS>([&](auto ic) __attribute__((always_inline)) {
        constexpr int i = decltype(ic)::value;
        if constexpr (i < NP) {
          constexpr int ss = i >> 2, db = i & 3;
          const u32x4_t pw = {pk[ss >> 1][4 * (ss & 1) + 0], pk[ss >> 1][4 * (ss & 1) + 1],
                              pk[ss >> 1][4 * (ss & 1) + 2], pk[ss >> 1][4 * (ss & 1) + 3]};
          o[db] = mfma32(opr[i % D], as_bf16x8(pw), o[db]);
        } else {
          constexpr int j = i - NP, kb = j & 1, ks = j >> 1;
          s[kb] = mfma32(opr[i % D], qf[ks], s[kb]);
        }
        if constexpr (i + D < NOPS) read(std::integral_constant<int, i + D>{});
        constexpr int GAP = NOPS / 8;
        if constexpr (i % GAP == GAP / 2) dma(i / GAP);
        __builtin_amdgcn_sched_barrier(0);
      });
    }
  };
  auto mfma_phase = [&](int t, const uint8_t* kb_t, const uint8_t* vb_prev, auto&& dma) __attribute__((always_inline)) {
    const bool pv = t >= 1 && (t - 1) * T::BN <= wmax;
    const bool qk = t < t_end && t * T::BN <= wmax;
    using Y = std::true_type;
    using N = std::false_type;
    if (pv && qk)
      mfma_block(Y{}, Y{}, kb_t, vb_prev, dma);
    else if (pv)
      mfma_block(Y{}, N{}, kb_t, vb_prev, dma);
    else if (qk)
      mfma_block(N{}, Y{}, kb_t, vb_prev, dma);
    else
      mfma_block(N{}, N{}, kb_t, vb_prev, dma);
  };

  if (t_end > 0) {
    // ring of NS stages: step t reads K(t) from kring[t % NS] and V(t-1) from vring[(t-1) % NS]; it fills
    // kring[(t-1) % NS] with K(t+NS-1) and vring[(t-2) % NS] with V(t+NS-2), whose previous contents were
    // last read in step t-1. Each step waits only for the loads issued NS-2 steps earlier. Group 0 issues
    // every load (DW = 4 per tile and wavefront); group 1 none.
    constexpr int PER_STEP = 2 * Dma<HD, PP_NW / 2>::DW;  // loads per group-0 wavefront per step
    static_assert(Dma<HD, PP_NW / 2>::DW == 4, "dma(j): j = 0..3 the K tile's loads, 4..7 the V tile's");
    auto step = [&](int t, const uint8_t* kb_t, uint8_t* kb_fill, const uint8_t* vb_prev, uint8_t* vb_fill) __attribute__((always_inline)) {
      // Group 0's loads of this step: K(t+NS-1) and V(t+NS-2). When both are whole tiles with 32-bit row offsets
      // (every step but the last one or two), each load is a per-lane offset added to a scalar tile base, issued
      // from inside the MFMA block without a branch; otherwise they go out before the block.
      const bool kload = t + NS - 1 < t_end, vload = t + NS - 2 < t_end;
      const int kk0 = (t + NS - 1) * T::BN, vk0 = (t + NS - 2) * T::BN;
      const bool inblock = kload && vload && kfast && vfast && kk0 + T::BN <= Nb && vk0 + T::BN <= Nb;
      const uint8_t* ksrc = reinterpret_cast<const uint8_t*>(Kb + (long long)kk0 * p.ksM);
      const uint8_t* vsrc = reinterpret_cast<const uint8_t*>(Vb + (long long)vk0 * p.vsM);
      constexpr int DW4 = Dma<HD, PP_NW / 2>::DW;
      auto dma = [&](int j) __attribute__((always_inline)) {
        const bool isk = j < DW4;
        const int i = isk ? j : j - DW4;
        // the offset passes through empty asm so that its 64-bit form is not kept live across the loop
        uint32_t o = isk ? kplan.off[i] : vplan.off[i];
        asm volatile("" : "+v"(o));
        const uint8_t* src = (isk ? ksrc : vsrc) + o;
        const uint32_t m0 = (uint32_t)reinterpret_cast<uintptr_t>(isk ? kb_fill : vb_fill) + (wu * DW4 + i) * 1024;
        asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(m0) : "memory");
      };
      auto no_dma = [](int) {};
      if (grp == 0 && !inblock) {
#pragma unroll
        for (int i = 0; i < DW4; ++i) {
          if (kload) kplan.template load_one<1>(i, kb_fill, Kb, p.ksM, kfast, kk0, Nb, w, lane);
          if (vload) vplan.template load_one<1>(i, vb_fill, Vb, p.vsM, vfast, vk0, Nb, w, lane);
        }
      }
      if (grp == 0 && inblock)
        mfma_phase(t, kb_t, vb_prev, dma);
      else if (grp == 0)
        mfma_phase(t, kb_t, vb_prev, no_dma);
      else if (t >= 1)
        softmax(t - 1);
      exec_barrier();  // staggers the two groups; no data passes here, so the loads issued above stay in flight
      if (grp == 0) {
        if (t < t_end) softmax(t);
      } else {
        mfma_phase(t, kb_t, vb_prev, no_dma);
      }
      // K(t+1) and V(t) must have landed: they were issued NS-2 steps ago (or in the prologue), and loads return
      // in issue order, so vmcnt((NS-2) * PER_STEP) leaves exactly the loads of the last NS-2 steps in flight.
      // That count is only right while every one of those steps issued its full PER_STEP loads, which holds
      // iff this step still issued a K load; near the end of the loop everything is drained instead.
      if (NS == 2 || t + NS - 1 >= t_end) {
        __builtin_amdgcn_s_waitcnt(0x0F70);
      } else if (NS == 3) {
        __builtin_amdgcn_s_waitcnt(vmcnt_le(PER_STEP));
      } else {
        __builtin_amdgcn_s_waitcnt(vmcnt_le(2 * PER_STEP));
      }
      __syncthreads();
    };
    // Steady state: steps 1 <= t <= t_fast in which both MFMA halves run, no row of this wavefront needs the mask
    // pass on tile t - 1 or t, and group 0's two loads are whole tiles with 32-bit row offsets. They run as pairs
    // (odd t, then even) of a straight-line body: buffers fixed at compile time, the load sources advanced by one
    // tile per step, no per-step flags. t_fast is per wavefront; every step, fast or not, has the same two
    // barriers, so the wavefronts stay in step.
    int t_fast = 0;
    // the fast steps form their load sources with 32-bit byte offsets from the tile bases (one scalar multiply
    // per tile instead of a 64-bit product): every wavefront runs this scalar arithmetic after the same barrier,
    // through the CU's one scalar unit
    const bool off32 = (long long)Nb * p.ksM * 2 < (1ll << 32) && (long long)Nb * p.vsM * 2 < (1ll << 32);
    if (MODE != MODE_VARLEN && kfast && vfast && off32) {
      const int lm = min(wmin, wmax);  // wmax < 0: no row of the wavefront sees a key
      t_fast = min(min(t_end - 2, Nb / T::BN - 2), lm >= T::BN - 1 ? (lm + 1) / T::BN - 1 : 0);
    }
    auto fast_step = [&](auto jc, int t, const uint8_t* ksrc, const uint8_t* vsrc) __attribute__((always_inline)) {
      constexpr int j = decltype(jc)::value;
      const uint8_t* kb_t = kring[j];
      uint8_t* kb_fill = kring[j ^ 1];
      const uint8_t* vb_prev = vring[j ^ 1];
      uint8_t* vb_fill = vring[j];
      constexpr int DW4 = Dma<HD, PP_NW / 2>::DW;
      auto dma = [&](int jj) __attribute__((always_inline)) {
        const bool isk = jj < DW4;
        const int i = isk ? jj : jj - DW4;
        uint32_t o = isk ? kplan.off[i] : vplan.off[i];
        asm volatile("" : "+v"(o));
        const uint8_t* src = (isk ? ksrc : vsrc) + o;
        const uint32_t m0 = (uint32_t)reinterpret_cast<uintptr_t>(isk ? kb_fill : vb_fill) + (wu * DW4 + i) * 1024;
        asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(m0) : "memory");
      };
      auto no_dma = [](int) {};
      using Y = std::true_type;
      using N = std::false_type;
      if (grp == 0)
        mfma_block(Y{}, Y{}, kb_t, vb_prev, dma);
      else
        softmax_core(N{}, (t - 1) * T::BN);
      exec_barrier();
      if (grp == 0)
        softmax_core(N{}, t * T::BN);
      else
        mfma_block(Y{}, Y{}, kb_t, vb_prev, no_dma);
      __builtin_amdgcn_s_waitcnt(0x0F70);
      __syncthreads();
    };
    static_assert(NS == 2, "the fast steps alternate two K/V buffers");
    // step t loads K(t+1) and V(t)
    const uint32_t ktile = (uint32_t)(T::BN * 2) * (uint32_t)p.ksM, vtile = (uint32_t)(T::BN * 2) * (uint32_t)p.vsM;
    auto ksrc_of = [&](int t) __attribute__((always_inline)) {
      return reinterpret_cast<const uint8_t*>(Kb) + (uint32_t)(t + 1) * ktile;
    };
    auto vsrc_of = [&](int t) __attribute__((always_inline)) {
      return reinterpret_cast<const uint8_t*>(Vb) + (uint32_t)t * vtile;
    };
    if constexpr (MODE == MODE_VARLEN) {
      for (int t = 0; t <= t_end; t += NS) {
#pragma unroll
        for (int j = 0; j < NS; ++j)
          if (t + j <= t_end)
            step(t + j, kring[j], kring[(j + NS - 1) % NS], vring[(j + NS - 1) % NS], vring[(j + NS - 2) % NS]);
      }
    } else {
    // step 0 (K(0) only), then pairs (odd t, t + 1)
    step(0, kring[0], kring[1], vring[1], vring[0]);
    for (int t = 1; t <= t_end; t += NS) {
      if (t + 1 <= t_fast) {
        fast_step(std::integral_constant<int, 1>{}, t, ksrc_of(t), vsrc_of(t));
        fast_step(std::integral_constant<int, 0>{}, t + 1, ksrc_of(t + 1), vsrc_of(t + 1));
        continue;
      }
      step(t, kring[1], kring[0], vring[0], vring[1]);
      if (t + 1 <= t_end) step(t + 1, kring[0], kring[1], vring[1], vring[0]);
    }
    }
  }

  // ---- epilogue: normalise, LSE, store
  const float l = halves_sum(l_run);
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  if (p.lse && rvalid && hf == 0) {
    int re = r;
    asm volatile("" : "+v"(re));  // the row's (token, head) recomputed here rather than kept across the loop
    const int te = re / p.G, ge = re - te * p.G;
    const float lse = l > 0.f ? (m_run + log2f(l)) * 0.69314718055994530942f : -INFINITY;
    p.lse[(long long)b * p.lsB + (long long)hk * p.lsH + (tok0 + te) * p.lsT + (long long)ge * p.lsG] = lse;
  }
  if (!p.o) return;
  if (o_vec == 2) {
    // through qo[w]: lane (lr, hf) writes 8 bytes of row lr per (db, q4); lane l then reads 16 bytes of row
    // 4i + l/16 and stores them: each store covers four whole rows
    uint8_t* ob = &qo[w][0];
    int ln = lane;
    asm volatile("" : "+v"(ln));  // addresses formed here, not kept live across the key loop
    const int lr2 = ln & 31, hf2 = ln >> 5;
    const uint32_t wa = (uint32_t)reinterpret_cast<uintptr_t>(ob) + lr2 * 256 + 8 * hf2, sw = swz(lr2);
#pragma unroll
    for (int db = 0; db < T::DB; ++db)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const uint32_t w0 = pack_bf16x2(o[db][4 * q4 + 0] * inv, o[db][4 * q4 + 1] * inv);
        const uint32_t w1 = pack_bf16x2(o[db][4 * q4 + 2] * inv, o[db][4 * q4 + 3] * inv);
        *reinterpret_cast<__attribute__((address_space(3))) u32x2_t*>(wa + ((((uint32_t)(4 * db + q4)) ^ sw) << 4)) =
            u32x2_t{w0, w1};
      }
    uint16_t* obase = p.o + (long long)b * p.osB + (long long)hk * p.osH + tok0 * p.osT;
    const int lrow0 = ln >> 4, pu = ln & 15;
    const int row0 = r0 + 32 * w + lrow0;
    int tq = row0 / p.G, gq = row0 - tq * p.G;
    const int d4 = 4 / p.G, m4 = 4 - d4 * p.G;
    // all eight reads first, so their LDS latencies overlap
    u32x4_t x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = *reinterpret_cast<const u32x4_t*>(ob + i * 1024 + 16 * lane);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = r0 + 32 * w + 4 * i + lrow0;
      const int u = pu ^ swz(4 * i + lrow0);
      if (row < Mb)
        __builtin_nontemporal_store(x[i], reinterpret_cast<u32x4_t*>(obase + (long long)tq * p.osT +
                                                                      (long long)gq * p.osG + 8 * u));
      tq += d4;
      gq += m4;
      if (gq >= p.G) { gq -= p.G; ++tq; }
    }
    return;
  }
  if (!rvalid) return;
  uint16_t* orow = p.o + (long long)b * p.osB + (long long)hk * p.osH + (tok0 + tok) * p.osT + (long long)g * p.osG;
#pragma unroll
  for (int db = 0; db < T::DB; ++db)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = 32 * db + 8 * q4 + 4 * hf;
      const uint32_t w0 = pack_bf16x2(o[db][4 * q4 + 0] * inv, o[db][4 * q4 + 1] * inv);
      const uint32_t w1 = pack_bf16x2(o[db][4 * q4 + 2] * inv, o[db][4 * q4 + 3] * inv);
      if (o_vec) {
        *reinterpret_cast<u32x2_t*>(orow + d) = u32x2_t{w0, w1};
      } else {
        *reinterpret_cast<uint32_t*>(orow + d) = w0;
        *reinterpret_cast<uint32_t*>(orow + d + 2) = w1;
      }
    }
  };  // item

  const int P = gridDim.x;
  if constexpr (MODE == MODE_VARLEN) {
    // packed sequences: the longest-first schedule of fmha_sched.h, computed alike by every workgroup
    vs_build<PP_BM>(vs, p.cu_seqlens, p.B, p.H, p.G, P, (int)blockIdx.x);
    if (vs.ok) {
      // round 0's item is known from the tables; the later rounds are worked out during its prologue
      const int first = vs_first(vs, P, (int)blockIdx.x);
      if (first < 0) {
        vs_rounds(vs, P, (int)blockIdx.x);
        __syncthreads();
      }
      for (int r = 0; r < vs.rounds; ++r) {
        const int v = r == 0 ? first : vs.mine[r];  // sequence * H + KV head, times 1024, plus row tile
        if (v < 0) continue;
        exec_barrier();  // as below
        item(v >> 10, v & 1023, r == 0);
      }
      return;
    }
  }
  for (int it = 0;; ++it) {
    long long vid;
    if (xcd_aware) {
      const int x = blockIdx.x & 7, m = blockIdx.x >> 3, PX = P >> 3;
      vid = 8ll * ((long long)it * PX + ((it & 1) ? PX - 1 - m : m)) + x;
    } else {
      vid = (long long)it * P + ((it & 1) ? P - 1 - (int)blockIdx.x : (int)blockIdx.x);
    }
    if (vid >= n_items) break;
    const int id = (int)vid;
    int bh, rank;
    if (xcd_aware) {
      const int per = BH >> 3, x = id & 7, j = id >> 3;
      bh = x + 8 * (j % per);
      rank = j / per;
    } else {
      bh = id % BH;
      rank = id / BH;
    }
    // every wavefront is done with the previous item's s_lim and K/V buffers (its last LDS read was followed by a
    // full barrier). Not __syncthreads(): its fence would wait for the previous item's output stores, whose
    // latency instead overlaps the next item's first loads.
    exec_barrier();
    item(bh, p.n_tiles - 1 - rank, false);
  }
}

// ------------------------------------------------------------------------------------------------------------
// Split-KV decode for short query blocks (at most 32 folded rows per (b, KV head)). The key range of each (b, KV
// head) is cut into num_splits splits of split_len keys; each split is streamed by P = 1, 2 or 4 wavefronts
// (p.wpsplit), each over its own part of split_len / P keys (a whole number of key tiles) through a private LDS
// region (a K and a V tile), so the loop has no workgroup barrier: the next K tile loads while the softmax and P.V
// of the current tile run, the next V tile while the next S^T runs. All G query heads of the KV head share each
// K/V tile. A workgroup's 4 wavefronts take 4 / P consecutive (b, split, KV head) tasks, KV head fastest, so with
// P = 1 they read neighbouring head slices of the same cache rows together. At the end the P partials of a split
// merge through LDS into the split's partial (O / l in fp32 and its natural-log LSE), which
// splitkv_combine_kernel merges across splits.
// A tile is 16 KB at either head dim: 64 keys at head_dim 128, 32 keys at head_dim 256.
// BLK0: the drop-in entry points' block rule (all rows of (b, h) form one block of at most 32 rows: when the
// largest raw qpos among them is 0, every live row sees key 0 only, reax_fmha_v8.cu:155-162, 224-235).
constexpr int DEC_NW = 4;

template <int HD>
struct DecTile {
  static constexpr int BN = HD == 128 ? 64 : 32;  // keys per tile
  static constexpr int NKB = BN / 32;             // 32-key blocks of S^T per tile
  static constexpr int NSS = BN / 16;             // 16-key MFMA steps of P.V per tile
  static constexpr int TILE = BN * HD * 2;        // 16 KB
  static constexpr int QK = HD / 16, DB = HD / 32;
  static_assert(TILE == 16384, "two 16 KB tiles per wavefront, four wavefronts: 128 KB of LDS");
};

template <int HD, bool BLK0>
__global__ void __launch_bounds__(256, 1) fmha_decode_kernel(const FwdParams p, int wpsplit) {
  using T = DecTile<HD>;
  // the K and V tiles of the four wavefronts; after the key loop the same bytes hold the partials being merged
  // (DEC_NW x 32 rows x HD fp32: 64 KB at head_dim 128, all 128 KB at 256)
  struct Lds {
    uint8_t k[DEC_NW][T::TILE];
    uint8_t v[DEC_NW][T::TILE];
  };
  static_assert(sizeof(Lds) >= DEC_NW * 32 * HD * sizeof(float), "merge area");
  __shared__ __align__(1024) Lds L;
  __shared__ float mm[DEC_NW * 32], lm[DEC_NW * 32];
  const int tid = threadIdx.x, lane = tid & 63, hf = lane >> 5, lr = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wavefront-uniform: keeps the loop control scalar
  const int P = wpsplit, part = w % P;
  const long long ntask = (long long)p.B * p.num_splits * p.H;
  const long long task = (long long)blockIdx.x * (DEC_NW / P) + w / P;
  const bool active = task < ntask;
  const long long tk = active ? task : 0;
  const int hk = (int)(tk % p.H);
  const int split = (int)((tk / p.H) % p.num_splits);
  const int b = (int)(tk / ((long long)p.H * p.num_splits));

  const int r = lr;  // row (folded: token r/G, head r%G); p.M <= 32
  const bool rvalid = r < p.M;
  const int tok = rvalid ? r / p.G : 0, g = rvalid ? r - tok * p.G : 0;
  const uint16_t* Kb = p.k + (long long)b * p.ksB + (long long)hk * p.ksH;
  const uint16_t* Vb = p.v + (long long)b * p.vsB + (long long)hk * p.vsH;
  const Dma<HD, 1, T::BN> kplan(p.ksM, 0, lane), vplan(p.vsM, 0, lane);
  const bool kfast = p.ksM * 2 * T::BN < (1ll << 31), vfast = p.vsM * 2 * T::BN < (1ll << 31);
  uint32_t kbase[T::NKB];
#pragma unroll
  for (int kb = 0; kb < T::NKB; ++kb) kbase[kb] = k_lane_base<HD>(kb, lr, hf);
  const uint32_t vbase = v_lane_base<HD>(lane);
  constexpr int DW = Dma<HD, 1, T::BN>::DW;
  // a decode split streams its keys once: nontemporal loads
  constexpr int LK = 2;
  uint8_t* kb_ = L.k[w];
  uint8_t* vb_ = L.v[w];
  const uint16_t* qrow = p.q + (long long)b * p.qsB + (long long)hk * p.qsH + (long long)tok * p.qsT + (long long)g * p.qsG;
  bf16x8_t qf[T::QK];
  // tiles t_beg .. t_end - 1; keys above a row's lim are masked; tile loads stop at kend
  int t_beg, t_end, kend, lim;
  {
    int qr = -1;
    if (rvalid && active) qr = p.qpos[(long long)b * p.qpBs + tok];
    if (BLK0 && p.N > 0 && wave_max(qr) == 0 && rvalid) qr = 0;  // the block rule: every live row sees key 0
    const int kbeg = split * p.split_len;
    kend = min(p.N, kbeg + p.split_len);
    const int qlen = p.split_len / P;  // a multiple of the tile size
    const int wbeg = kbeg + part * qlen;
    kend = min(kend, wbeg + qlen);
    lim = max(min(qr, kend - 1), -1);
    if (lim < wbeg) lim = -1;
    const int wmax = __builtin_amdgcn_readfirstlane(wave_max(lim));
    t_beg = wbeg / T::BN;
    t_end = wmax < wbeg ? t_beg : wmax / T::BN + 1;
    // the first K tile, then Q, then the first V tile: one memory latency for all three. Loads return in issue
    // order, so the explicit wait for K(t_beg) before the first S^T (at most the V tile's DW loads outstanding)
    // also covers Q; the waits the compiler adds for Q, which does not count the tile loads, are only stricter.
    if (t_end > t_beg) kplan.template tile<2>(kb_, Kb, p.ksM, kfast, t_beg * T::BN, kend, 0, lane);
#pragma unroll
    for (int ks = 0; ks < T::QK; ++ks)
      qf[ks] = as_bf16x8(rvalid ? ld16(qrow + 16 * ks + 8 * hf) : u32x4_t{0u, 0u, 0u, 0u});
    if (t_end > t_beg) vplan.template tile<2>(vb_, Vb, p.vsM, vfast, t_beg * T::BN, kend, 0, lane);
  }
  const int wmin = __builtin_amdgcn_readfirstlane(wave_min(lim));

  f32x16_t o[T::DB];
#pragma unroll
  for (int db = 0; db < T::DB; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[db][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const float cc = p.scale_log2;
  f32x16_t s[T::NKB];
  uint32_t pk[T::NKB][8];

  for (int t = t_beg; t < t_end; ++t) {
    const int k0 = t * T::BN, kn = k0 + T::BN;  // this tile's first key, the next tile's
    const bool more = t + 1 < t_end;
    __builtin_amdgcn_s_waitcnt(vmcnt_le(DW));  // K(t) landed (V(t) may be in flight)
#pragma unroll
    for (int kb = 0; kb < T::NKB; ++kb) {
#pragma unroll
      for (int e = 0; e < 16; ++e) s[kb][e] = 0.f;
#pragma unroll
      for (int ks = 0; ks < T::QK; ++ks) {
        const u32x4_t kf = *reinterpret_cast<const u32x4_t*>(kb_ + (kbase[kb] ^ (32u * ks)));
        s[kb] = mfma32(as_bf16x8(kf), qf[ks], s[kb]);
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the K tile has been read
    if (more) kplan.template tile<LK>(kb_, Kb, p.ksM, kfast, kn, kend, 0, lane);
    if (k0 + T::BN - 1 > wmin) {
#pragma unroll
      for (int kb = 0; kb < T::NKB; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = k0 + 32 * kb + 8 * (v >> 2) + 4 * hf + (v & 3);
          if (key > lim) s[kb][v] = -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < T::NKB; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[kb][v]);
    mx = halves_max(mx) * cc;
    if (__any(mx > m_run + RESCALE_SLACK)) {
      const float m_new = fmaxf(m_run, mx);
      // before the wavefront's first admitted key every row's O and sum are still 0: nothing to rescale (with
      // one or two tiles per wavefront, the 64 accumulator multiplies are a visible part of the loop)
      if (__any(m_run != -INFINITY)) {
        const float alpha = m_new == -INFINITY ? 1.0f : fast_exp2(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < T::DB; ++db)
#pragma unroll
          for (int e = 0; e < 16; ++e) o[db][e] *= alpha;
      }
      m_run = m_new;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    float ps[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < T::NKB; ++kb)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float p0 = fast_exp2(__builtin_fmaf(s[kb][2 * i], cc, -m_use));
        const float p1 = fast_exp2(__builtin_fmaf(s[kb][2 * i + 1], cc, -m_use));
        ps[(i & 1) * 2] += p0;
        ps[(i & 1) * 2 + 1] += p1;
        pk[kb][i] = pack_bf16x2(p0, p1);
      }
    l_run += (ps[0] + ps[1]) + (ps[2] + ps[3]);
    if (more)
      __builtin_amdgcn_s_waitcnt(vmcnt_le(DW));  // V(t) landed, K(t+1) may be in flight
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_le(0));
#pragma unroll
    for (int ss = 0; ss < T::NSS; ++ss) {
      const u32x4_t pw = {pk[ss >> 1][4 * (ss & 1) + 0], pk[ss >> 1][4 * (ss & 1) + 1], pk[ss >> 1][4 * (ss & 1) + 2],
                          pk[ss >> 1][4 * (ss & 1) + 3]};
      const bf16x8_t pb = as_bf16x8(pw);
#pragma unroll
      for (int db = 0; db < T::DB; ++db) o[db] = mfma32(v_operand<HD>(vb_, db, ss, vbase), pb, o[db]);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the V tile has been read
    if (more) vplan.template tile<LK>(vb_, Vb, p.vsM, vfast, kn, kend, 0, lane);
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_le(0));

  const float l = halves_sum(l_run);
  // ---- merge the P partials of each split through LDS (the tile buffers are free once every wavefront is here)
  __syncthreads();
  // [DEC_NW][32 rows][HD], 16-byte groups of row x XOR-swizzled by x & 15: a wavefront's stores of 4 dims of its
  // 32 rows, and the merge's reads along a row, spread over the banks (unswizzled, the rows' equal dims share a
  // bank: 32-way conflicts, ~2 us per merge)
  float* om = reinterpret_cast<float*>(&L);
  auto omx = [](int x, int d) { return x * HD + (d ^ ((x & 15) << 2)); };
#pragma unroll
  for (int db = 0; db < T::DB; ++db)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int d = 32 * db + 8 * q4 + 4 * hf;
      *reinterpret_cast<f32x4_t*>(om + omx(w * 32 + lr, d)) =
          f32x4_t{o[db][4 * q4 + 0], o[db][4 * q4 + 1], o[db][4 * q4 + 2], o[db][4 * q4 + 3]};
    }
  if (hf == 0) {
    mm[w * 32 + lr] = l > 0.f ? m_run : -INFINITY;
    lm[w * 32 + lr] = l;
  }
  __syncthreads();
  if (!active) return;
  const int w0 = w - part;  // first wavefront of this split's group
  const long long prow0 = ((long long)(b * p.H + hk) * p.num_splits + split) * p.M;
  for (int idx = part * 64 + lane; idx < p.M * HD; idx += P * 64) {
    const int row = idx / HD, d = idx - row * HD;
    float mx = -INFINITY;
    for (int ww = w0; ww < w0 + P; ++ww) mx = fmaxf(mx, mm[ww * 32 + row]);
    float lsum = 0.f, acc = 0.f;
    if (mx != -INFINITY) {
      for (int ww = w0; ww < w0 + P; ++ww) {
        const float mw = mm[ww * 32 + row];
        const float f = mw == -INFINITY ? 0.f : fast_exp2(mw - mx);
        lsum += f * lm[ww * 32 + row];
        acc += f * om[omx(ww * 32 + row, d)];
      }
    }
    p.ws_o[(prow0 + row) * HD + d] = lsum > 0.f ? acc / lsum : 0.f;
    if (d == 0) p.ws_lse[prow0 + row] = lsum > 0.f ? (mx + log2f(lsum)) * 0.69314718055994530942f : -INFINITY;
  }
}

// LSE-weighted merge of the split partials: NW = 1 or 4 wavefronts per (b, kv head, row), 4 / NW rows per workgroup.
//   lse = log(sum_s exp(lse_s)),  O = sum_s exp(lse_s - lse) * O_s     (O_s already normalised by its row sum)
// Wavefront w of a row merges splits w, w + NW, w + 2 NW, ...: lane j holds the LSE of its j-th split (64 per pass),
// the wavefronts' maxima meet in LDS, and the partial rows are read in batches of BATCH independent loads per lane
// (the first batch issued before the LSEs are known), so a row costs two or three memory round trips rather than one
// per split; the wavefronts' sums meet in LDS again. Four wavefronts per row pay when there are many splits (the
// drop-in decode at batch 1: 128 splits, 7.5 us against 13 us with one), one when there are few (config 4: 16).
__device__ __forceinline__ float wave_maxf(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x = fmaxf(x, __shfl_xor(x, off, 64));
  return x;
}
__device__ __forceinline__ float wave_sumf(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

constexpr int CMB_WAVES = 4;  // wavefronts per workgroup of the combine kernel

// POST: the drop-in reax_fmha_qp's epilogue instead of the O / LSE store (reax_fmha_v11.cu:451-522): O rounded to
// bf16, times the bf16 sigmoid of the gate qg[R][hq][HD + d], rounded once, stored to out[R][hq * HD + d] for the
// token row R = inv[b * Lq + token]; rows with R < 0 are left untouched.
template <int HD, bool POST, int CMB_NW>
__global__ void __launch_bounds__(64 * CMB_WAVES) splitkv_combine_kernel(const FwdParams p) {
  static_assert(CMB_NW == 1 || CMB_NW == CMB_WAVES, "one or all wavefronts of the workgroup per row");
  constexpr int DPL = HD / 64;  // dims per lane
  constexpr int BATCH = 16;
  __shared__ float red[CMB_WAVES][DPL][64];
  __shared__ float rsum[CMB_WAVES], rmax[CMB_WAVES];
  const int lane = threadIdx.x & 63, wg = threadIdx.x >> 6;
  const int w = wg % CMB_NW, w0 = wg - w;  // this wavefront's index within its row, the row's first wavefront
  const long long row_id = (long long)blockIdx.x * (CMB_WAVES / CMB_NW) + wg / CMB_NW;
  const bool live = row_id < (long long)p.B * p.H * p.M;
  const int r = (int)(row_id % p.M);
  const long long bh = row_id / p.M;
  const int b = (int)(bh / p.H), hk = (int)(bh % p.H);
  const int S = p.num_splits;
  const long long base = bh * S * p.M + r;                  // split s's partial row: base + s * M
  const int Sw = S > w ? (S - w + CMB_NW - 1) / CMB_NW : 0;  // this wavefront's splits: w + CMB_NW j, j < Sw
  auto prow = [&](int j) -> const float* {
    return p.ws_o + (base + (long long)(w + CMB_NW * j) * p.M) * HD + DPL * lane;
  };
  auto load_batch = [&](float (&v)[BATCH][DPL], int i0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < BATCH; ++i) {
      const float* po = prow(min(i0 + i, Sw - 1));  // past the end: a clamped (in-bounds) row, weighted 0
      if constexpr (DPL == 4) {
        const f32x4_t x = *reinterpret_cast<const f32x4_t*>(po);
#pragma unroll
        for (int e = 0; e < DPL; ++e) v[i][e] = x[e];
      } else {
#pragma unroll
        for (int e = 0; e < DPL; ++e) v[i][e] = po[e];
      }
    }
  };
  float v[BATCH][DPL];
  const int Sl = live ? Sw : 0;  // a workgroup's last rows may lie past the end: they merge nothing
  if (Sl > 0) load_batch(v, 0);
  float l0 = lane < Sl ? p.ws_lse[base + (long long)(w + CMB_NW * lane) * p.M] : -INFINITY;
  float mloc = l0;
  for (int j0 = 64; j0 < Sl; j0 += 64)
    if (j0 + lane < Sl) mloc = fmaxf(mloc, p.ws_lse[base + (long long)(w + CMB_NW * (j0 + lane)) * p.M]);
  mloc = wave_maxf(mloc);
  float mx = mloc;
  if constexpr (CMB_NW > 1) {
    if (lane == 0) rmax[wg] = mloc;
    __syncthreads();
    mx = rmax[w0];
#pragma unroll
    for (int i = 1; i < CMB_NW; ++i) mx = fmaxf(mx, rmax[w0 + i]);
  }
  float acc[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) acc[e] = 0.f;
  float wsum = 0.f;
  if (mx != -INFINITY) {
    for (int j0 = 0; j0 < Sl; j0 += 64) {
      const int n = min(64, Sl - j0);
      const float lv = j0 == 0 ? l0 : (lane < n ? p.ws_lse[base + (long long)(w + CMB_NW * (j0 + lane)) * p.M] : -INFINITY);
      const float wl = lane < n ? fast_exp2((lv - mx) * 1.44269504088896340736f) : 0.f;
      wsum += wl;
      for (int i0 = 0; i0 < n; i0 += BATCH) {
        if (j0 + i0 > 0) load_batch(v, j0 + i0);
#pragma unroll
        for (int i = 0; i < BATCH; ++i) {
          const float wi = i0 + i < n ? __shfl(wl, min(i0 + i, 63), 64) : 0.f;
#pragma unroll
          for (int e = 0; e < DPL; ++e) acc[e] += wi * v[i][e];
        }
      }
    }
  }
  wsum = wave_sumf(wsum);
  if constexpr (CMB_NW > 1) {
#pragma unroll
    for (int e = 0; e < DPL; ++e) red[wg][e][lane] = acc[e];
    if (lane == 0) rsum[wg] = wsum;
    __syncthreads();
    if (w != 0) return;
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[e] = (red[w0][e][lane] + red[w0 + 1][e][lane]) + (red[w0 + 2][e][lane] + red[w0 + 3][e][lane]);
    wsum = (rsum[w0] + rsum[w0 + 1]) + (rsum[w0 + 2] + rsum[w0 + 3]);
  }
  if (!live) return;
  const float inv = wsum > 0.f ? 1.0f / wsum : 0.f;
  const int tok = r / p.G, g = r - tok * p.G;
  if (POST) {
    const int R = p.inv[(long long)b * p.Lq + tok];
    if (R < 0) return;
    const long long hq = (long long)hk * p.G + g;
    const uint16_t* grow = p.qg + (long long)R * p.qg_rs + hq * (2 * HD) + HD + DPL * lane;
    uint16_t* orow = p.outp + (long long)R * p.out_rs + hq * HD + DPL * lane;
#pragma unroll
    for (int j = 0; j < DPL; j += 2) {
      const uint32_t gw = *reinterpret_cast<const uint32_t*>(grow + j);
      const uint32_t ob = pack_bf16x2(acc[j] * inv, acc[j + 1] * inv);
      const uint32_t s0 = sigmoid_bf16_bits(gw & 0xffffu), s1 = sigmoid_bf16_bits(gw >> 16);
      *reinterpret_cast<uint32_t*>(orow + j) = pack_bf16x2(bf16lo(ob) * bf16lo(s0), bf16hi(ob) * bf16lo(s1));
    }
    return;
  }
  if (p.lse && lane == 0)
    p.lse[(long long)b * p.lsB + (long long)hk * p.lsH + (long long)tok * p.lsT + (long long)g * p.lsG] =
        wsum > 0.f ? mx + logf(wsum) : -INFINITY;
  uint16_t* orow = p.o + (long long)b * p.osB + (long long)hk * p.osH + (long long)tok * p.osT + (long long)g * p.osG;
#pragma unroll
  for (int j = 0; j < DPL; j += 2)
    *reinterpret_cast<uint32_t*>(orow + DPL * lane + j) = pack_bf16x2(acc[j] * inv, acc[j + 1] * inv);
}

// ------------------------------------------------------------------------------------------------ host side


template <int HD, int MODE, bool POST, bool SPLIT>
static int launch_fwd_t(const FwdParams& p, hipStream_t stream) {
  using T = FwdTile<HD>;
  const long long nwg = (long long)p.B * p.H * p.n_tiles * (SPLIT ? p.num_splits : 1);
  if (nwg <= 0 || nwg > INT_MAX) return (int)hipErrorInvalidConfiguration;
  const int o_vec8 = (!POST && p.o) ? (aligned_elems(p.o, 4, {p.osB, p.osH, p.osT, p.osG}) ? 1 : 0) : 0;
  hipLaunchKernelGGL((fmha_fwd_kernel<HD, MODE, POST, SPLIT>), dim3((unsigned)nwg), dim3(T::NT), 0, stream, p, o_vec8);
  return (int)hipGetLastError();
}

// Argument checks shared by every forward entry point; fills the derived fields.
static int prepare(FwdParams& p, bool post) {
  // Input rows are read with 16-byte loads: bases and row strides must be multiples of 8 elements (the
  // reference's cp.async has the same precondition, v8:169, 183, 191). O needs even strides (v8:396-397).
  if (!p.q || !p.k || !p.v) return (int)hipErrorInvalidValue;
  if (!aligned_elems(p.q, 8, {p.qsB, p.qsH, p.qsT, p.qsG}) || !aligned_elems(p.k, 8, {p.ksB, p.ksH, p.ksM}) ||
      !aligned_elems(p.v, 8, {p.vsB, p.vsH, p.vsM}))
    return (int)hipErrorInvalidValue;
  if (p.o && !aligned_elems(p.o, 2, {p.osB, p.osH, p.osT, p.osG})) return (int)hipErrorInvalidValue;
  if (post && (!p.inv || !p.qg || !p.outp || !aligned_elems(p.qg, 4, {p.qg_rs}) || !aligned_elems(p.outp, 4, {p.out_rs})))
    return (int)hipErrorInvalidValue;
  if (p.G <= 0 || p.B < 0 || p.H < 0 || p.M < 0 || p.N < 0) return (int)hipErrorInvalidValue;
  p.scale_log2 = p.scale * 1.44269504088896340736f;
  p.n_tiles = (int)(((long long)p.M + FwdTile<128>::BM - 1) / FwdTile<128>::BM);
  return 0;
}

// Compute units of the device that owns `stream` (the current device for the null stream), cached per device: the
// persistent kernels launch one workgroup per CU. Entries are atomics, so concurrent first calls from several host
// threads at worst query the attribute twice and store the same value.
int device_cus(hipStream_t stream) {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (stream ? hipStreamGetDevice(stream, &dev) != hipSuccess : hipGetDevice(&dev) != hipSuccess) return 0;
  if (dev < 0 || dev >= 64) return 0;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 0;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

template <int MODE>
static int launch_fwd_pp(FwdParams p, hipStream_t stream) {
  p.n_tiles = (int)(((long long)p.M + PP_BM - 1) / PP_BM);
  const long long n_items = (long long)p.B * p.H * p.n_tiles;
  if (n_items <= 0 || n_items > INT_MAX) return (int)hipErrorInvalidConfiguration;
  const int cus = device_cus(stream);
  if (cus <= 0) return (int)hipErrorInvalidDevice;
  const long long nwg = n_items < cus ? n_items : cus;  // one workgroup per CU (its LDS and registers fill one)
  // output stores: 2 whole rows staged through LDS (16-byte aligned rows), 1 eight-byte, 0 four-byte pieces
  const int o_vec = !p.o ? 0
                    : aligned_elems(p.o, 8, {p.osB, p.osH, p.osT, p.osG}) ? 2
                    : aligned_elems(p.o, 4, {p.osB, p.osH, p.osT, p.osG}) ? 1 : 0;
  hipLaunchKernelGGL((fmha_fwd_pp_kernel<MODE, PP_STAGES>), dim3((unsigned)nwg), dim3(64 * PP_NW), 0, stream, p, o_vec);
  return (int)hipGetLastError();
}

// ------------------------------------------------------------------------------------------------------------
// Row-block prefill for small head_dim-128 qpos calls (reax_fmha_qx at S 512: the ping-pong kernel's 256-row items
// would fill 16 of 256 CUs). The task is a 32-row block (b, block, KV head), blocks with the most keys first, one
// 8-wavefront workgroup per block: wavefront w takes the 32-key tiles w, w + 8, ... of the block's key range
// [0, its largest key limit], each through its own 8 KB K and V buffers (the next tile's K loads as soon as the
// current S^T has read K, its V after P.V). Two wavefronts per SIMD: while one waits for its tile copies (the CU's
// vector memory path carries the heaviest block's whole K/V range, 256 KB at S 512), the other computes. Q crosses
// once through LDS (one 1 KB copy per wavefront). The eight partials merge through the tile buffers: each
// wavefront, as its key loop ends, writes its partial into its own buffers; after one barrier wavefront w
// finalises the 8 values per lane of dim block w / 2, half w % 2, weighting and adding the eight partials' slices
// (128 KB through LDS).
constexpr int RB_NW = 8;
constexpr int RB_BN = 32;

__global__ void __launch_bounds__(64 * RB_NW, 1) fmha_rows_kernel(const FwdParams p, int o_vec8) {
  constexpr int HD = 128, BN = RB_BN, TILE = BN * HD * 2, QK = HD / 16, DB = HD / 32;
  using DmaT = Dma<HD, 1, BN>;
  constexpr int DW = DmaT::DW;  // 8 loads per tile
  struct Lds {
    uint8_t k[RB_NW][TILE];
    uint8_t v[RB_NW][TILE];
  };
  // after its key loop a wavefront's K and V buffers hold its partial for the merge: 16 slots of 64 x 16 bytes
  static_assert(TILE == 8 * 1024, "8 merge slots per tile buffer");
  __shared__ __align__(1024) Lds L;
  __shared__ __align__(1024) uint8_t qs[32 * HD * 2];  // the block's Q rows, swizzled as a 32-row K tile
  __shared__ float mm[RB_NW * 32], lm[RB_NW * 32];
  const int tid = threadIdx.x, lane = tid & 63, hf = lane >> 5, lr = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nrb = (p.M + 31) / 32;
  const unsigned t32 = blockIdx.x, bhn = (unsigned)p.B * (unsigned)p.H;  // blockIdx.x < B * nrb * H
  const int hk = (int)(t32 % (unsigned)p.H);
  const int b = (int)((t32 / (unsigned)p.H) % (unsigned)p.B);
  const int rb = nrb - 1 - (int)(t32 / bhn);
  const int r = rb * 32 + lr;
  const bool rvalid = r < p.M;
  const int tok = rvalid ? r / p.G : 0, g = rvalid ? r - tok * p.G : 0;
  const uint16_t* Kb = p.k + (long long)b * p.ksB + (long long)hk * p.ksH;
  const uint16_t* Vb = p.v + (long long)b * p.vsB + (long long)hk * p.vsH;
  const DmaT kplan(p.ksM, 0, lane), vplan(p.vsM, 0, lane);
  const bool kfast = p.ksM * 2 * BN < (1ll << 31), vfast = p.vsM * 2 * BN < (1ll << 31);
  uint8_t* kb_ = L.k[w];
  uint8_t* vb_ = L.v[w];
  {
    // Q copy w: rows 4w .. 4w + 3 of the block (lane l: row 4w + l / 16, logical unit (l % 16) ^ swz(row)); rows
    // past the end read the last row (never stored)
    const int lrow = 4 * w + (lane >> 4), pu = lane & 15;
    const int rr = min(rb * 32 + lrow, p.M - 1);
    const int tq = rr / p.G, gq = rr - tq * p.G;
    const uint16_t* src = p.q + (long long)b * p.qsB + (long long)hk * p.qsH + (long long)tq * p.qsT +
                          (long long)gq * p.qsG + 8 * (pu ^ swz(lrow));
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)reinterpret_cast<uintptr_t>(&qs[w * 1024]));
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(m0) : "memory");
  }
  // the first tile does not depend on qpos: its K and V go out with Q, then qpos (loads complete in issue order,
  // and the wait the compiler puts before qpos's use, which does not count the copies, drains them all)
  if (w * BN < p.N) {
    kplan.template tile<1>(kb_, Kb, p.ksM, kfast, w * BN, p.N, 0, lane);
    vplan.template tile<1>(vb_, Vb, p.vsM, vfast, w * BN, p.N, 0, lane);
  }
  int qr = -1;
  if (rvalid) qr = p.qpos[(long long)b * p.qpBs + tok];
  const int lim = max(min(qr, p.N - 1), -1);
  const int blim = wave_ext_dpp<true>(lim);  // every wavefront holds the same 32 rows
  const int wmin = wave_ext_dpp<false>(lim);
  const int t_end = blim < 0 ? 0 : blim / BN + 1;  // key tiles any row of the block sees
  __builtin_amdgcn_s_waitcnt(0x0F70);              // vmcnt(0): this wavefront's Q copy (and its first tile)
  __syncthreads();                                 // ... and every other wavefront's Q copy
  bf16x8_t qf[QK];
  {
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const uint32_t qa = (uint32_t)reinterpret_cast<uintptr_t>(&qs[0]) + k_lane_base<HD>(0, ln & 31, ln >> 5);
#pragma unroll
    for (int ks = 0; ks < QK; ++ks)
      qf[ks] = as_bf16x8(*reinterpret_cast<const __attribute__((address_space(3))) u32x4_t*>(qa ^ (32u * ks)));
  }
  const uint32_t kbase = k_lane_base<HD>(0, lr, hf);
  const uint32_t vbase = v_lane_base<HD>(lane);

  f32x16_t o[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[db][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const float cc = p.scale_log2;
  f32x16_t s;
  uint32_t pk[8];
  for (int t = w; t < t_end; t += RB_NW) {
    const int k0 = t * BN, kn = k0 + RB_NW * BN;
    const bool more = t + RB_NW < t_end;
    __builtin_amdgcn_s_waitcnt(vmcnt_le(DW));  // K(t) landed (V(t) may be in flight)
#pragma unroll
    for (int e = 0; e < 16; ++e) s[e] = 0.f;
#pragma unroll
    for (int ks = 0; ks < QK; ++ks) {
      const u32x4_t kf = *reinterpret_cast<const u32x4_t*>(kb_ + (kbase ^ (32u * ks)));
      s = mfma32(as_bf16x8(kf), qf[ks], s);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the K tile has been read
    if (more) kplan.template tile<1>(kb_, Kb, p.ksM, kfast, kn, p.N, 0, lane);
    if (k0 + BN - 1 > wmin) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int key = k0 + 8 * (v >> 2) + 4 * hf + (v & 3);
        if (key > lim) s[v] = -INFINITY;
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[v]);
    mx = halves_max(mx) * cc;
    if (__any(mx > m_run + RESCALE_SLACK)) {
      const float m_new = fmaxf(m_run, mx);
      if (__any(m_run != -INFINITY)) {  // before the first admitted key O and the sums are still 0
        const float alpha = m_new == -INFINITY ? 1.0f : fast_exp2(m_run - m_new);
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int e = 0; e < 16; ++e) o[db][e] *= alpha;
      }
      m_run = m_new;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    float ps[2] = {0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float p0 = fast_exp2(__builtin_fmaf(s[2 * i], cc, -m_use));
      const float p1 = fast_exp2(__builtin_fmaf(s[2 * i + 1], cc, -m_use));
      ps[i & 1] += p0 + p1;
      pk[i] = pack_bf16x2(p0, p1);
    }
    l_run += ps[0] + ps[1];
    if (more)
      __builtin_amdgcn_s_waitcnt(vmcnt_le(DW));  // V(t) landed, K(t+8) may be in flight
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_le(0));
#pragma unroll
    for (int ss = 0; ss < 2; ++ss) {
      const bf16x8_t pb = as_bf16x8(u32x4_t{pk[4 * ss], pk[4 * ss + 1], pk[4 * ss + 2], pk[4 * ss + 3]});
#pragma unroll
      for (int db = 0; db < DB; ++db) o[db] = mfma32(v_operand<HD>(vb_, db, ss, vbase), pb, o[db]);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the V tile has been read
    if (more) vplan.template tile<1>(vb_, Vb, p.vsM, vfast, kn, p.N, 0, lane);
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_le(0));

  // ---- merge: O = sum_w f_w O_w / L, f_w = 2^(m_w - M), M = max_w m_w, L = sum_w f_w l_w. As soon as its key
  // loop ends, wavefront w writes its unweighted partial into its own tile buffers (free now, and read by no
  // other wavefront): slice d (dim block d / 2, values 8 (d % 2) .. + 7 of each lane's 16, finalised by
  // wavefront d) as two 16-byte pieces per lane in 1 KB slot 2 d + q (slots 0-7 in its K buffer, 8-15 in its V
  // buffer; consecutive lanes 16 bytes apart), its own slice included. One barrier, then wavefront w weights and
  // adds the eight slices of slot 2 w + q, with no per-wavefront branch or register selection.
  const float l = halves_sum(l_run);
  if (hf == 0) {
    mm[w * 32 + lr] = l > 0.f ? m_run : -INFINITY;
    lm[w * 32 + lr] = l;
  }
  auto slot = [&](int src, int sl) __attribute__((always_inline)) {
    return reinterpret_cast<u32x4_t*>(sl < 8 ? &L.k[src][sl * 1024] : &L.v[src][(sl - 8) * 1024]) + lane;
  };
#pragma unroll
  for (int d = 0; d < RB_NW; ++d) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const f32x16_t& od = o[d >> 1];
      const int v0 = 8 * (d & 1) + 4 * q;
      *slot(w, 2 * d + q) = u32x4_t{__float_as_uint(od[v0]), __float_as_uint(od[v0 + 1]),
                                    __float_as_uint(od[v0 + 2]), __float_as_uint(od[v0 + 3])};
    }
  }
  __syncthreads();  // every partial, row maximum and sum visible
  // all slice reads first, so that their LDS latencies overlap each other and the row maxima's
  u32x4_t sl[RB_NW][2];
#pragma unroll
  for (int src = 0; src < RB_NW; ++src)
#pragma unroll
    for (int q = 0; q < 2; ++q) sl[src][q] = *slot(src, 2 * w + q);
  float ms[RB_NW], ls[RB_NW];
#pragma unroll
  for (int src = 0; src < RB_NW; ++src) {
    ms[src] = mm[src * 32 + lr];
    ls[src] = lm[src * 32 + lr];
  }
  float M = -INFINITY;
#pragma unroll
  for (int src = 0; src < RB_NW; ++src) M = fmaxf(M, ms[src]);
  float fin[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float Lsum = 0.f;
#pragma unroll
  for (int src = 0; src < RB_NW; ++src) {
    const float f = ms[src] == -INFINITY ? 0.f : fast_exp2(ms[src] - M);  // every row maximum -inf: all f are 0
    Lsum += f * ls[src];
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) fin[4 * q + e] = __builtin_fmaf(f, __uint_as_float(sl[src][q][e]), fin[4 * q + e]);
  }
  const float inv = Lsum > 0.f ? 1.0f / Lsum : 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) fin[e] *= inv;
  if (!rvalid) return;
  if (p.lse && w == 0 && hf == 0)
    p.lse[(long long)b * p.lsB + (long long)hk * p.lsH + (long long)tok * p.lsT + (long long)g * p.lsG] =
        Lsum > 0.f ? (M + log2f(Lsum)) * 0.69314718055994530942f : -INFINITY;
  if (!p.o) return;
  // values 8 (w % 2) + 4 q + e of dim block w / 2 are dims 32 (w / 2) + 8 (2 (w % 2) + q) + 4 hf + e: one 8-byte
  // piece per q (two 4-byte pieces when rows are only 4-byte aligned)
  uint16_t* orow = p.o + (long long)b * p.osB + (long long)hk * p.osH + (long long)tok * p.osT +
                   (long long)g * p.osG + 32 * (w >> 1) + 16 * (w & 1) + 4 * hf;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const uint32_t w0 = pack_bf16x2(fin[4 * q + 0], fin[4 * q + 1]);
    const uint32_t w1 = pack_bf16x2(fin[4 * q + 2], fin[4 * q + 3]);
    // ordinary stores: each wavefront writes 32 bytes of a row, and the L2 merges the eight wavefronts' pieces into
    // whole lines (as nontemporal stores the pieces reach HBM separately: 1.55 MB written instead of 1.04)
    if (o_vec8) {
      *reinterpret_cast<u32x2_t*>(orow + 8 * q) = u32x2_t{w0, w1};
    } else {
      reinterpret_cast<uint32_t*>(orow + 8 * q)[0] = w0;
      reinterpret_cast<uint32_t*>(orow + 8 * q)[1] = w1;
    }
  }
}

// The row-block kernel (head_dim 128, qpos mode): one 8-wavefront workgroup per 32-row block.
static int launch_fwd_rows(const FwdParams& p, hipStream_t stream) {
  const long long nwg = (long long)p.B * p.H * ((p.M + 31) / 32);
  if (nwg <= 0 || nwg > INT_MAX) return (int)hipErrorInvalidConfiguration;
  const int o_vec8 = p.o && aligned_elems(p.o, 4, {p.osB, p.osH, p.osT, p.osG}) ? 1 : 0;  // 8-byte output pieces
  hipLaunchKernelGGL(fmha_rows_kernel, dim3((unsigned)nwg), dim3(64 * RB_NW), 0, stream, p, o_vec8);
  return (int)hipGetLastError();
}

int launch_fwd(const FwdParams& p0, int head_dim, int mode, bool post, hipStream_t stream) {
  FwdParams p = p0;
  if (const int rc = prepare(p, post)) return rc;
  // head_dim 128 qpos prefills whose 256-row items would occupy at most a quarter of the CUs (config 1: 16 items):
  // 32-row blocks with their keys split over 8 wavefronts, 8 times the workgroups of the ping-pong kernel
  if (head_dim == 128 && !post && !p.qpos0_block && mode == MODE_QPOS) {
    const long long pp_items = (long long)p.B * p.H * (((long long)p.M + PP_BM - 1) / PP_BM);
    if (pp_items > 0) {
      const int cus = device_cus(stream);
      if (cus > 0 && pp_items * 4 <= cus) return launch_fwd_rows(p, stream);
    }
  }
  // head_dim 128 qpos / varlen without the POST epilogue: the ping-pong kernel once a row tile has enough rows
  // to fill both groups (short query blocks, e.g. decode, keep the 4-wavefront kernel); it has no drop-in block
  // rule (qpos0_block), which the 4-wavefront, pair and decode kernels implement
  if (head_dim == 128 && !post && !p.qpos0_block && p.M > FwdTile<128>::BM) {
    if (mode == MODE_QPOS) return launch_fwd_pp<MODE_QPOS>(p, stream);
    if (mode == MODE_VARLEN) return launch_fwd_pp<MODE_VARLEN>(p, stream);
  }
  // the drop-in entry points at short query blocks (decode steps): key splits across the GPU when worthwhile
  if (head_dim == 256 && mode == MODE_QPOS && p.qpos0_block && p.M <= 32) {
    const int rc = launch_short_split(p, post, stream);
    if (rc != SHORT_NOT_TAKEN) return rc;
  }
  // head_dim 256 qpos / varlen (the drop-in shape, with or without the POST epilogue): the wavefront-pair
  // ping-pong kernel once there are rows for both of its groups (fmha_fwd_pair.hip)
  if (head_dim == 256 && (mode == MODE_QPOS || (mode == MODE_VARLEN && !post)) && p.M > 64)
    return launch_fwd_pair(p, mode, post, stream);
  // head_dim 128 is reached only through the extension entry points (qpos or varlen, no gate, no bias); the
  // drop-in entry points (bias, POST, block rule) run at head_dim 256
  if (head_dim == 128) {
    if (post || p.qpos0_block) return (int)hipErrorInvalidValue;
    if (mode == MODE_QPOS) return launch_fwd_t<128, MODE_QPOS, false, false>(p, stream);
    if (mode == MODE_VARLEN) return launch_fwd_t<128, MODE_VARLEN, false, false>(p, stream);
  } else if (head_dim == 256) {
    if (mode == MODE_QPOS)
      return post ? launch_fwd_t<256, MODE_QPOS, true, false>(p, stream) : launch_fwd_t<256, MODE_QPOS, false, false>(p, stream);
    if (mode == MODE_BIAS && !post) return launch_fwd_t<256, MODE_BIAS, false, false>(p, stream);
    if (mode == MODE_VARLEN && !post) return launch_fwd_t<256, MODE_VARLEN, false, false>(p, stream);
  }
  return (int)hipErrorInvalidValue;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t splitkv_workspace_bytes(int B, int H, int M, int head_dim, int num_splits) {
  if (B <= 0 || H <= 0 || M <= 0 || num_splits <= 0 || (head_dim != 128 && head_dim != 256)) return 0;
  const size_t rows = (size_t)B * H * num_splits * M;
  return align256(rows * head_dim * sizeof(float)) + align256(rows * sizeof(float));
}

// Key-split parameters of the decode kernel for num_splits requested splits over N keys: P wavefronts per split
// (each streaming at least DEC_MIN_TILES tiles when the split is long enough) and split_len, a multiple of P tiles.
static void decode_split_shape(int head_dim, int N, int num_splits, int& P, int& split_len) {
  constexpr int DEC_MIN_TILES = 8;
  const int BN = head_dim == 128 ? DecTile<128>::BN : DecTile<256>::BN;
  const int q = (N + num_splits - 1) / num_splits;
  const int qt = max(1, (q + BN - 1) / BN);
  P = qt >= 4 * DEC_MIN_TILES ? 4 : qt >= 2 * DEC_MIN_TILES ? 2 : 1;
  split_len = ((qt + P - 1) / P) * P * BN;
}

// The combine kernel for p.num_splits splits: four wavefronts per row from 32 splits on, else one.
static int launch_combine(const FwdParams& p, int head_dim, bool post, hipStream_t stream) {
  const long long rows = (long long)p.B * p.H * p.M;
  const bool wide = p.num_splits >= 32;
  const long long nwg = wide ? rows : (rows + CMB_WAVES - 1) / CMB_WAVES;
  if (nwg <= 0 || nwg > INT_MAX) return (int)hipErrorInvalidConfiguration;
  const dim3 grid((unsigned)nwg), block(64 * CMB_WAVES);
  if (head_dim == 128 && !post) {
    if (wide) hipLaunchKernelGGL((splitkv_combine_kernel<128, false, CMB_WAVES>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((splitkv_combine_kernel<128, false, 1>), grid, block, 0, stream, p);
  } else if (head_dim == 256 && post) {
    if (wide) hipLaunchKernelGGL((splitkv_combine_kernel<256, true, CMB_WAVES>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((splitkv_combine_kernel<256, true, 1>), grid, block, 0, stream, p);
  } else if (head_dim == 256) {
    if (wide) hipLaunchKernelGGL((splitkv_combine_kernel<256, false, CMB_WAVES>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((splitkv_combine_kernel<256, false, 1>), grid, block, 0, stream, p);
  } else {
    return (int)hipErrorInvalidValue;
  }
  return (int)hipGetLastError();
}

int launch_decode_split(FwdParams p, int head_dim, int P, bool post, hipStream_t stream) {
  const long long ntask = (long long)p.B * p.H * p.num_splits;
  const long long nwg = (ntask + (DEC_NW / P) - 1) / (DEC_NW / P);
  if (nwg <= 0 || nwg > INT_MAX) return (int)hipErrorInvalidConfiguration;
  if (head_dim == 128) {
    if (post || p.qpos0_block) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL((fmha_decode_kernel<128, false>), dim3((unsigned)nwg), dim3(256), 0, stream, p, P);
  } else if (p.qpos0_block) {
    hipLaunchKernelGGL((fmha_decode_kernel<256, true>), dim3((unsigned)nwg), dim3(256), 0, stream, p, P);
  } else {
    hipLaunchKernelGGL((fmha_decode_kernel<256, false>), dim3((unsigned)nwg), dim3(256), 0, stream, p, P);
  }
  if (const int rc = (int)hipGetLastError()) return rc;
  return launch_combine(p, head_dim, post, stream);
}

void set_workspace(FwdParams& p, void* ws, int head_dim) {
  const size_t rows = (size_t)p.B * p.H * p.num_splits * p.M;
  p.ws_o = reinterpret_cast<float*>(ws);
  p.ws_lse = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(ws) + align256(rows * head_dim * sizeof(float)));
}

int launch_splitkv(const SplitParams& sp, int head_dim, hipStream_t stream) {
  FwdParams p = sp.f;
  if (const int rc = prepare(p, false)) return rc;
  if (!p.o || sp.num_splits <= 0 || !sp.ws) return (int)hipErrorInvalidValue;
  if (!aligned_elems(p.o, 2, {p.osB, p.osH, p.osT, p.osG})) return (int)hipErrorInvalidValue;
  const size_t need = splitkv_workspace_bytes(p.B, p.H, p.M, head_dim, sp.num_splits);
  if (need == 0 || sp.ws_bytes < need || (reinterpret_cast<uintptr_t>(sp.ws) & 255u)) return (int)hipErrorInvalidValue;
  p.num_splits = sp.num_splits;
  set_workspace(p, sp.ws, head_dim);
  if ((head_dim == 128 || head_dim == 256) && p.M <= 32) {
    // wavefront-split decode kernel: P wavefronts per split
    int P;
    decode_split_shape(head_dim, p.N, sp.num_splits, P, p.split_len);
    return launch_decode_split(p, head_dim, P, false, stream);
  }
  const int per = (p.N + sp.num_splits - 1) / sp.num_splits;
  p.split_len = ((per + FwdTile<128>::BN - 1) / FwdTile<128>::BN) * FwdTile<128>::BN;
  if (p.split_len <= 0) p.split_len = FwdTile<128>::BN;
  int rc = head_dim == 128 ? launch_fwd_t<128, MODE_QPOS, false, true>(p, stream)
         : head_dim == 256 ? launch_fwd_t<256, MODE_QPOS, false, true>(p, stream)
                           : (int)hipErrorInvalidValue;
  if (rc) return rc;
  return launch_combine(p, head_dim, false, stream);
}

}  // namespace reax
