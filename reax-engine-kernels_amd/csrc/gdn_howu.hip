// Gated-DeltaNet chunked forward for gfx950. Replaces howu3_skip / reax_howu / howu3_dense / howu3_smem,
// libreax_howu/reax_howu.cu:349-376 (kernel howu3_kernel, reax_howu.cu:55-347), and reax_howu_norm,
// libreax_howu/reax_howu_norm_v3.cu:431-435 (kernel howu3p_kernel: the same with a fused gated-RMSNorm epilogue).
//
// Per sequence and value head hv (key head hv / (HV/H)), with the state h [128 k-dims][128 v-dims] (fp32, from 0)
// and per 64-token chunk (g: chunk-local cumulative log2 decay, eg = 2^g; A: the chunk solve's bf16 output):
//   vb = bf16(v beta), kb = bf16(bf16(k beta) eg)                                                 (howu:95-104, 146-156)
//   ub = bf16(A vb), wb = bf16(A kb)        (skip form: the blocks of A above the diagonal blocks read as 0)
//   AQ[t][s] = bf16((q_t . k_s) 2^(g_t - g_s)) for s <= t (both in the chunk), else 0                (howu:165-196)
//   vw = wb bf16(h), oi = q bf16(h); x = ub - vw; vn = bf16(x); vdec = bf16(x 2^(g_last - g_t))      (howu:210-244)
//   o = bf16(fma(AQ vn, scale, (oi 2^(g_t)) scale))                                                 (howu:256-283)
//   h = h 2^(g_last) + k^T vdec                                                                     (howu:285-300)
// Gated-norm epilogue (reax_howu_norm, norm_v3:276-392): o is not stored; a token with output row R = f2s[token]
// (R < 0: skipped) writes out[R][hv][c] = bf16(bf16(w[c] bf16(o[c] rr)) silu(z[R][hv][c])), rr = 1 / sqrt(sum(o^2)
// factor + eps) with the sum formed per 4 columns ((o0^2 + o1^2) + o2^2) + o3^2 and then over the 32 groups by a
// halving tree (norm_v3:352-358), silu(z) = z / (1 + exp(-z)) in fp32. rr and exp are evaluated to fp32 accuracy
// where the reference uses rsqrtf and expf.
// Every bf16 rounding point and elementwise operation follows the reference; the matrix products accumulate in fp32
// on the matrix cores in the hardware's order, as the reference's tensor-core products do in theirs, so results
// agree to bf16 accuracy, not bit for bit.
//
// Layout for MI355X: one workgroup of 4 wavefronts per (sequence, value head), as the reference's one CTA, with the
// 128 x 128 state in the accumulators: wavefront w owns v-dims 32 w .. 32 w + 31 of it. Every product is a
// v_mfma_f32_32x32x16_bf16 sequence; the products that involve the state or the chunk's x = u - w h (w h, q h,
// AQ vn, k^T vdec) take that operand straight from the wavefront's own accumulators (bf16 pairs and one
// v_permlane32_swap per pair to reach the MFMA's k order), so the state never goes through LDS. A chunk's q, k, v
// and A are copied from HBM straight into LDS (global_load_lds_dwordx4) one chunk ahead, into the other of two
// buffer sets, so the copy overlaps the current chunk's products; operands whose k runs down the stored rows are
// read with ds_read_b64_tr_b16, and products whose results feed other wavefronts are computed transposed where
// that lets each lane store 4 adjacent bf16 at once. Two barriers per chunk.
#include <hip/hip_runtime.h>
#include <stdint.h>

#pragma GCC visibility push(default)
#include "libreax_howu.h"
#pragma GCC visibility pop

#include "fmha_tiles.h"

namespace reax {
namespace {

constexpr int HW_BT = 64, HW_D = 128, HW_THREADS = 256;

// Row swizzles. 256-byte rows (q, k, v / vb, kb, wb): unit u of row r at ((u ^ swz(r)) << 4), the attention
// kernels' K/V layout (fragment reads of 16 consecutive rows and transposed reads of 4 rows x 4 units are both
// free of bank conflicts). 128-byte rows (A, AQ; two rows per 256-byte bank line): unit u of row r at
// ((u ^ sw8(r)) << 4), which puts 16 consecutive rows' units in 16 distinct bank groups.
__device__ __forceinline__ int sw8(int r) { return (r ^ (r >> 3)) & 7; }
__device__ __forceinline__ int off256(int r, int u) { return r * 256 + ((u ^ swz(r)) << 4); }
__device__ __forceinline__ int off128(int r, int u) { return r * 128 + ((u ^ sw8(r)) << 4); }

// One chunk's inputs as copied from HBM (q, k, v rows of 128 bf16, A rows of 64) and its per-token scalars.
struct HowuSet {
  uint16_t q[HW_BT * HW_D];
  uint16_t k[HW_BT * HW_D];
  uint16_t v[HW_BT * HW_D];  // turned into vb = bf16(v beta) in place before the chunk's products
  uint16_t a[HW_BT * HW_BT];
  float g[HW_BT], eg[HW_BT], beta[HW_BT], da[HW_BT];  // g, 2^g, beta, 2^(g_last - g) (0 past the chunk's end)
};
struct HowuLds {
  HowuSet set[2];              // chunk i computes from set[i & 1] while chunk i + 1 is copied into the other
  uint16_t kb[HW_BT * HW_D];   // [s][d] bf16(bf16(k beta) 2^g)
  uint16_t wb[HW_BT * HW_D];   // [t][d] bf16(A kb); the norm epilogue stages o here
  uint16_t aq[HW_BT * HW_BT];  // [t][s]
};

// Inputs past a sequence's end and A's blocks above the diagonal blocks are copied from here: 16 zero bytes.
__device__ __align__(16) uint32_t howu_zero[4];

__device__ __forceinline__ float bf16_val(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ float bf16_round(float x) { return __uint_as_float(pack_bf16x2(x, 0.f) << 16); }

// Workgroup barrier once this wavefront's LDS accesses have completed, leaving its vector-memory operations (the
// next chunk's copies, output stores) in flight.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ void wait_vm() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// Direct global -> LDS copy of 16 bytes per lane (lane l's bytes land at lds + 16 l). Without a memory clobber the
// compiler may move other LDS accesses across it: the destination buffer set is neither read nor written between
// the copy and prep()'s wait, which does clobber memory.
// NT adds the nontemporal hint, for data read exactly once (v and A; q and k serve two value heads).
template <bool NT = false>
__device__ __forceinline__ void dma16(const void* src, uint8_t* lds) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)reinterpret_cast<uintptr_t>(lds));
  if (NT)
    asm volatile("global_load_lds_dwordx4 %0, off nt" ::"v"(src), "{m0}"(m0));
  else
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(m0));
}

// MFMA operand (a 32-wide block of m or n, 16 k) from LDS rows of 256 bytes: row `row` (the lane's m or n), the
// lane's 8 consecutive k at unit 2 ks + (lane / 32).
__device__ __forceinline__ bf16x8_t frag256(const uint16_t* buf, int row, int ks, int hf) {
  return as_bf16x8(*reinterpret_cast<const u32x4_t*>(reinterpret_cast<const uint8_t*>(buf) + off256(row, 2 * ks + hf)));
}
__device__ __forceinline__ bf16x8_t frag128(const uint16_t* buf, int row, int ks, int hf) {
  return as_bf16x8(*reinterpret_cast<const u32x4_t*>(reinterpret_cast<const uint8_t*>(buf) + off128(row, 2 * ks + hf)));
}

// MFMA operand whose k runs down the rows of a 256-byte-row buffer [k][x]: x = 32 db + lane % 32, k rows of step ks,
// read with two ds_read_b64_tr_b16 (in each 16-lane group lane i reads 4 x-values of row i / 4 and receives row
// 0..3's values of x-value i). NAT: lane half hf gets k = 16 ks + 8 hf + 0..7 (the MFMA's own k order); otherwise
// k = 16 ks + 4 hf + {0..3, 8..11}, the order of a 32 x 32 accumulator's rows, so that the other operand can be taken
// from accumulators as they are (any k order serves as long as both operands share it).
template <bool NAT>
__device__ __forceinline__ bf16x8_t tr_frag(const uint16_t* buf, int db, int ks, int lane) {
  const int i = lane & 15, dh = (lane >> 4) & 1, hf = lane >> 5;
  u32x2_t part[2];
#pragma unroll
  for (int sec = 0; sec < 2; ++sec) {
    const int row = 16 * ks + (NAT ? 8 * hf + 4 * sec : 4 * hf + 8 * sec) + (i >> 2);
    const int unit = 4 * db + 2 * dh + ((i >> 1) & 1);
    part[sec] = ds_read_tr16(reinterpret_cast<const uint8_t*>(buf) + off256(row, unit) + 8 * (i & 1));
  }
  return as_bf16x8(u32x4_t{part[0][0], part[0][1], part[1][0], part[1][1]});
}

// MFMA operand over rows 16 s .. 16 s + 15 of a 32 x 32 fp32 accumulator tile (its rows are the operand's k, the
// lane's column its m or n), rounded to bf16. NAT: in the MFMA's k order, which takes one exchange with the lane 32
// away per register pair (v_permlane32_swap: lanes 0-31 hold rows 16 s + {0..3, 8..11}, lanes 32-63 rows
// 16 s + {4..7, 12..15}); otherwise in the accumulator's own row order (pairs with tr_frag<false>).
template <bool NAT>
__device__ __forceinline__ bf16x8_t acc_frag(const f32x16_t& a, int s) {
  const uint32_t p0 = pack_bf16x2(a[8 * s + 0], a[8 * s + 1]), p1 = pack_bf16x2(a[8 * s + 2], a[8 * s + 3]);
  const uint32_t p2 = pack_bf16x2(a[8 * s + 4], a[8 * s + 5]), p3 = pack_bf16x2(a[8 * s + 6], a[8 * s + 7]);
  if (!NAT) return as_bf16x8(u32x4_t{p0, p1, p2, p3});
  const auto r0 = __builtin_amdgcn_permlane32_swap(p0, p2, false, false);
  const auto r1 = __builtin_amdgcn_permlane32_swap(p1, p3, false, false);
  return as_bf16x8(u32x4_t{r0[0], r1[0], r0[1], r1[1]});
}

// z / (1 + exp(-z)) in fp32 for the gated norm: |z| < 64 by 2^(-z log2 e) with the exponent split into an exact
// 16-significant-bit product and a small remainder (second-order correction), about 5 ulp; otherwise with exp in
// double precision (1 + exp(-z) rounded to fp32, infinite on overflow, then an IEEE division)
__device__ __forceinline__ float silu_f32(float z) {
  if (!(z > -64.0f && z < 64.0f)) return z / (float)(1.0 + exp(-(double)z));
  const float zr = __uint_as_float(__float_as_uint(z) & 0xffff0000u);  // bf16 part: exact product with H below
  const float a_hi = zr * -1.44268798828125f;
  const float a_lo = (z - zr) * -1.44269504088896340736f + zr * -7.052607543300837e-06f;
  const float t = a_lo * 0.6931471824645996f;
  const float eh = fast_exp2(a_hi);
  const float e = __builtin_fmaf(eh, __builtin_fmaf(0.5f * t, t, t), eh);
  return z * __builtin_amdgcn_rcpf(1.0f + e);
}

struct NormArgs {
  const int* f2s;
  const uint16_t* z;
  long long ZS;
  const uint16_t* nw;
  float eps, factor;
};

template <bool DENSE, bool NORM>
__global__ void __launch_bounds__(HW_THREADS, 1) howu_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                                             const uint16_t* __restrict__ v,
                                                             const uint16_t* __restrict__ beta,
                                                             const uint16_t* __restrict__ Ag, const float* __restrict__ g,
                                                             uint16_t* __restrict__ o, const int64_t* __restrict__ cu,
                                                             float scale, int NSEQ, int H, int HV, const NormArgs na) {
  __shared__ __align__(16) HowuLds S;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, l32 = lane & 31, hf = lane >> 5;
  // Workgroups are dealt to the 8 XCDs in turn (workgroup b to XCD b % 8). The GQ value heads of one key head are
  // placed on one XCD, so that their shared q and k rows are read from HBM once and then hit that XCD's L2.
  const int GQ = HV / H;
  int item = (int)blockIdx.x;
  if (GQ > 1) {
    const int full = (NSEQ * HV) / (8 * GQ) * (8 * GQ);
    if (item < full) item = (((item >> 3) / GQ) * 8 + (item & 7)) * GQ + (item >> 3) % GQ;
  }
  const int i_n = NSEQ - 1 - item / HV, hv = item % HV, kh = hv / GQ;
  const long long bos = cu[i_n];
  const int T = (int)(cu[i_n + 1] - bos);
  const int nch = (T + HW_BT - 1) / HW_BT;

  // Copies: wavefront wv fills rows 16 wv .. 16 wv + 15 of q, k, v (four 1 KB direct-to-LDS loads each: rows
  // 16 wv + 4 i + lane / 16) and of A (two loads: rows 16 wv + 8 i + lane / 8); lane l of a load lands at byte
  // 16 l of it, i.e. at a swizzled unit of its row, and fetches the unit the swizzle puts there.
  uint32_t off_qk[4], off_v[4], off_a[2];
  int row_a[2], unit_a[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 16 * wv + 4 * i + (lane >> 4), u = (lane & 15) ^ swz(r);
    off_qk[i] = (uint32_t)(r * H * 256 + 16 * u);
    off_v[i] = (uint32_t)(r * HV * 256 + 16 * u);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = 16 * wv + 8 * i + (lane >> 3), u = (lane & 7) ^ sw8(r);
    row_a[i] = r;
    unit_a[i] = u;
    off_a[i] = (uint32_t)(r * HV * 128 + 16 * u);
  }
  const uint8_t* zero = reinterpret_cast<const uint8_t*>(howu_zero);
  float g_next = 0.f;  // g and beta (bits) of token `lane` of the chunk being copied
  uint16_t b_next = 0;

  // Chunk c's copies in four parts (0: q, 1: k, 2: v, 3: A, g and beta), issued at points spread over the current
  // chunk's products: every workgroup reaches the same point at about the same time, and a burst of all of them
  // held the issuing wavefronts for as long as HBM took to deliver it.
  auto issue = [&](int c, HowuSet& st, int part) {
    const int t0 = c * HW_BT, nv = min(HW_BT, T - t0);
    if (part < 3) {
      const uint16_t* src = part == 2 ? v + ((bos + t0) * HV + hv) * HW_D : (part ? k : q) + ((bos + t0) * H + kh) * HW_D;
      uint16_t* dst = part == 2 ? st.v : part ? st.k : st.q;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool ok = 16 * wv + 4 * i + (lane >> 4) < nv;
        const uint8_t* from = ok ? reinterpret_cast<const uint8_t*>(src) + (part == 2 ? off_v[i] : off_qk[i]) : zero;
        if (part == 2)
          dma16<true>(from, reinterpret_cast<uint8_t*>(dst) + (4 * wv + i) * 1024);
        else
          dma16<false>(from, reinterpret_cast<uint8_t*>(dst) + (4 * wv + i) * 1024);
      }
      return;
    }
    const uint8_t* ab = reinterpret_cast<const uint8_t*>(Ag + ((bos + t0) * HV + hv) * HW_BT);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      // the skip form reads A's blocks above the diagonal 16 x 16 blocks as zeros
      const bool ok = row_a[i] < nv && (DENSE || (unit_a[i] >> 1) <= (row_a[i] >> 4));
      dma16<true>(ok ? ab + off_a[i] : zero, reinterpret_cast<uint8_t*>(st.a) + (2 * wv + i) * 1024);
    }
    // g and beta of token `lane` (rows past the end read the last token's; prep() zeroes them). Unconditional
    // loads whose results are first used after the copies have landed: a masked load or a conversion here would
    // make the compiler wait for it, and the vector-memory counter only counts down in order, so that wait would
    // also wait for every copy issued above.
    const long long row = (bos + t0 + min(lane, nv - 1)) * HV + hv;
    g_next = g[row];
    b_next = beta[row];
  };
  // Once chunk c's copies have landed: its scalars, then vb = bf16(v beta) in place and kb = bf16(bf16(k beta) 2^g),
  // each wavefront on the 16 rows it copied itself (so no barrier is needed between its copies and this pass).
  auto prep = [&](int c, HowuSet& st) {
    wait_vm();
    const int nv = min(HW_BT, T - c * HW_BT);
    const float glast = __shfl(g_next, nv - 1);
    if ((lane >> 4) == wv) {
      const bool ok = lane < nv;
      const float gg = ok ? g_next : 0.f;
      st.g[lane] = gg;
      st.eg[lane] = fast_exp2(gg);
      st.beta[lane] = ok ? bf16_val(b_next) : 0.f;
      st.da[lane] = ok ? fast_exp2(glast - gg) : 0.f;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * wv + 4 * i + (lane >> 4), byte = r * 256 + 16 * (lane & 15);
      const float b = st.beta[r], e = st.eg[r];
      const u32x4_t vw = *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const uint8_t*>(st.v) + byte);
      const u32x4_t kw = *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const uint8_t*>(st.k) + byte);
      u32x4_t vo, ko;
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        vo[x] = pack_bf16x2(bf16lo(vw[x]) * b, bf16hi(vw[x]) * b);
        ko[x] = pack_bf16x2(bf16_round(bf16lo(kw[x]) * b) * e, bf16_round(bf16hi(kw[x]) * b) * e);
      }
      *reinterpret_cast<u32x4_t*>(reinterpret_cast<uint8_t*>(st.v) + byte) = vo;
      *reinterpret_cast<u32x4_t*>(reinterpret_cast<uint8_t*>(S.kb) + byte) = ko;
    }
  };

  // The state h [128 k-dims][128 v-dims]: wavefront wv holds v-dims 32 wv .. 32 wv + 31 of all k-dims, tile j =
  // k-dims 32 j .. 32 j + 31 (accumulator layout: column = v-dim, rows = k-dims).
  f32x16_t h[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) h[j][e] = 0.f;
  u32x2_t opend[2][4];  // the last chunk's o (bf16), stored after the next chunk's copies are issued
  int t0_prev = 0, nv_prev = 0;
  auto store_o = [&](int tt) {  // rows 32 tt .. 32 tt + 31 of the last chunk's o
    const int t = 32 * tt + (lane & 31);
    if (t < nv_prev) {
      uint16_t* orow = o + ((bos + t0_prev + t) * HV + hv) * HW_D + 32 * wv + 4 * hf;
#pragma unroll
      for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x2_t*>(orow + 8 * j) = opend[tt][j];
    }
  };

  if (nch > 0) {
    for (int part = 0; part < 4; ++part) issue(0, S.set[0], part);
    prep(0, S.set[0]);
  }
  for (int c = 0; c < nch; ++c) {
    HowuSet& st = S.set[c & 1];
    const int t0 = c * HW_BT, nv = min(HW_BT, T - t0);
    __syncthreads();  // chunk c's copies, scalars, vb and kb are visible; every wavefront is done with chunk c - 1
    // The lane index passes through an empty asm so that the compiler derives the per-lane LDS addresses here,
    // where they are used, instead of holding ~100 of them in registers across the loop.
    int ln = tid & 63;
    asm volatile("" : "+v"(ln));
    const int lane = ln, l32 = ln & 31, hf = ln >> 5;
    const bool more = c + 1 < nch;
    HowuSet& nx = S.set[(c + 1) & 1];
    if (more) issue(c + 1, nx, 0);

    // ---- ub = bf16(A vb) for v-dims 32 wv.. (rows t, kept in registers) and wb = bf16(A kb) for k-dims 32 wv..,
    // computed transposed (rows d, column t) -> wb[t][d]. Both take A's rows as fragments (row t = 32 tt + l32,
    // s = 16 ks + 8 hf + 0..7); in the skip form rows 0..31 have no s >= 32.
    constexpr int KS0 = DENSE ? 4 : 2;
    f32x16_t ub[2];
    {
      bf16x8_t vf[4], kf[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        vf[ks] = tr_frag<true>(st.v, wv, ks, lane);
        kf[ks] = tr_frag<true>(S.kb, wv, ks, lane);
      }
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        f32x16_t au = {}, aw = {};
#pragma unroll
        for (int ks = 0; ks < (tt ? 4 : KS0); ++ks) {
          const bf16x8_t af = frag128(st.a, 32 * tt + l32, ks, hf);
          au = mfma32(af, vf[ks], au);
          aw = mfma32(kf[ks], af, aw);
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) ub[tt][e] = bf16_round(au[e]);
        const int t = 32 * tt + l32;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          *reinterpret_cast<u32x2_t*>(reinterpret_cast<uint8_t*>(S.wb) + off256(t, 4 * wv + j) + 8 * hf) =
              u32x2_t{pack_bf16x2(aw[4 * j], aw[4 * j + 1]), pack_bf16x2(aw[4 * j + 2], aw[4 * j + 3])};
        if (tt == 0 && !NORM && c > 0) store_o(0);
        if (tt == 1 && more) issue(c + 1, nx, 1);
      }
    }
    // ---- AQ[t][s] = bf16((q_t . k_s) 2^(g_t - g_s)) for s <= t < nv, else 0: wavefronts 0-2 take the 32 x 32
    // tiles (s-block, t-block) (0, 0), (0, 1), (1, 1), computed transposed (rows s, column t) -> aq[t][s]. The
    // tile (1, 0) is all zeros and never read.
    if (wv < 3) {
      const int sb = wv == 2 ? 1 : 0, tb = wv == 0 ? 0 : 1;
      f32x16_t acc = {};
#pragma unroll
      for (int kd = 0; kd < 8; ++kd)
        acc = mfma32(frag256(st.k, 32 * sb + l32, kd, hf), frag256(st.q, 32 * tb + l32, kd, hf), acc);
      const int t = 32 * tb + l32;
      const float gt = st.g[t];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int s0 = 32 * sb + 8 * j + 4 * hf;
        const f32x4_t gs = *reinterpret_cast<const f32x4_t*>(st.g + s0);
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = (s0 + e <= t && t < nv) ? acc[4 * j + e] * fast_exp2(gt - gs[e]) : 0.f;
        *reinterpret_cast<u32x2_t*>(reinterpret_cast<uint8_t*>(S.aq) + off128(t, 4 * sb + j) + 8 * hf) =
            u32x2_t{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
      }
    }
    lds_barrier();  // wb and AQ complete

    // ---- vw = wb bf16(h) and (q bf16(h))^T for v-dims 32 wv.., one 16-deep slice of k-dims at a time: bf16(h) as
    // an MFMA operand straight from the state's accumulators (B of w h, A of (q h)^T)
    f32x16_t vw[2] = {}, oi[2] = {};
#pragma unroll
    for (int kd = 0; kd < 8; ++kd) {
      if (kd == 2 && !NORM && c > 0) store_o(1);
      if (kd == 5 && more) issue(c + 1, nx, 2);
      const bf16x8_t hb = acc_frag<true>(h[kd >> 1], kd & 1);
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        vw[tt] = mfma32(frag256(S.wb, 32 * tt + l32, kd, hf), hb, vw[tt]);
        oi[tt] = mfma32(hb, frag256(st.q, 32 * tt + l32, kd, hf), oi[tt]);
      }
    }
    // ---- x = ub - vw; vn = bf16(x), vdec = bf16(x 2^(g_last - g_t)) as operands of (AQ vn)^T and k^T vdec
    bf16x8_t vnf[4], vdf[4];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      f32x16_t x, xd;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4_t da = *reinterpret_cast<const f32x4_t*>(st.da + 32 * tt + 8 * j + 4 * hf);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[4 * j + e] = ub[tt][4 * j + e] - vw[tt][4 * j + e];
          xd[4 * j + e] = x[4 * j + e] * da[e];
        }
      }
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        vnf[2 * tt + s] = acc_frag<true>(x, s);
        vdf[2 * tt + s] = acc_frag<false>(xd, s);
      }
    }
    if (more) issue(c + 1, nx, 3);
    // ---- o^T (rows v-dims 32 wv.., column t) = scale (AQ vn)^T + scale 2^(g_t) (q bf16(h))^T
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      f32x16_t av = {};
#pragma unroll
      for (int ks = 0; ks < 2 * (tt + 1); ++ks) av = mfma32(vnf[ks], frag128(S.aq, 32 * tt + l32, ks, hf), av);
      const float egt = st.eg[32 * tt + l32];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float r[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = __builtin_fmaf(av[4 * j + e], scale, (oi[tt][4 * j + e] * egt) * scale);
        opend[tt][j] = u32x2_t{pack_bf16x2(r[0], r[1]), pack_bf16x2(r[2], r[3])};
      }
    }
    t0_prev = t0;
    nv_prev = nv;
    // ---- h = h 2^(g_last) + k^T vdec
    const float gl = fast_exp2(st.g[nv - 1]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int e = 0; e < 16; ++e) h[j][e] = h[j][e] * gl;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) h[j] = mfma32(tr_frag<false>(st.k, j, ks, lane), vdf[ks], h[j]);
    }

    if (NORM) {
      lds_barrier();  // every wavefront is done reading wb
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          *reinterpret_cast<u32x2_t*>(reinterpret_cast<uint8_t*>(S.wb) + off256(32 * tt + l32, 4 * wv + j) + 8 * hf) =
              opend[tt][j];
      lds_barrier();
      // two rows per wavefront at a time, one per 32-lane half: lane l of a half holds columns 4l .. 4l+3
#pragma unroll 1
      for (int i = 0; i < HW_BT / 8; ++i) {
        const int t = 2 * (wv * (HW_BT / 8) + i) + hf;
        const int R = t < nv ? na.f2s[bos + t0 + t] : -1;
        if (R < 0) continue;  // the same for the whole half
        const u32x2_t xo =
            *reinterpret_cast<const u32x2_t*>(reinterpret_cast<const uint8_t*>(S.wb) + off256(t, l32 >> 1) + 8 * (l32 & 1));
        const float x[4] = {bf16lo(xo[0]), bf16hi(xo[0]), bf16lo(xo[1]), bf16hi(xo[1])};
        float p = ((x[0] * x[0] + x[1] * x[1]) + x[2] * x[2]) + x[3] * x[3];
#pragma unroll
        for (int d = 16; d >= 1; d >>= 1) p = p + __shfl_down(p, d, 32);
        const float tot = __shfl(p, 0, 32);
        const float rr = (float)(1.0 / sqrt((double)(tot * na.factor + na.eps)));
        const u32x2_t wv2 = *reinterpret_cast<const u32x2_t*>(na.nw + 4 * l32);
        const u32x2_t zv = *reinterpret_cast<const u32x2_t*>(na.z + (long long)R * na.ZS + hv * HW_D + 4 * l32);
        const float w[4] = {bf16lo(wv2[0]), bf16hi(wv2[0]), bf16lo(wv2[1]), bf16hi(wv2[1])};
        const float zz[4] = {bf16lo(zv[0]), bf16hi(zv[0]), bf16lo(zv[1]), bf16hi(zv[1])};
        float res[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float y = bf16_round(x[e] * rr);
          const float y2 = bf16_round(w[e] * y);
          res[e] = y2 * silu_f32(zz[e]);
        }
        *reinterpret_cast<u32x2_t*>(o + ((long long)R * HV + hv) * HW_D + 4 * l32) =
            u32x2_t{pack_bf16x2(res[0], res[1]), pack_bf16x2(res[2], res[3])};
      }
    }
    if (c + 1 < nch) prep(c + 1, S.set[(c + 1) & 1]);
  }
  if (!NORM && nch > 0) {
    store_o(0);
    store_o(1);
  }
}

template <bool DENSE, bool NORM = false>
int launch_howu(const void* q, const void* k, const void* v, const void* beta, const void* A, const void* g, void* o,
                const void* cu, float scale, int N, int H, int HV, void* stream, const NormArgs na = {}) {
  // an empty grid: the reference's launch fails with the invalid-configuration error
  if (N <= 0 || HV <= 0) return (int)hipErrorInvalidConfiguration;
  // the key head of value head hv is hv / (HV / H): H must divide HV (the reference divides by zero otherwise);
  // missing or misaligned buffers (its 16-byte cp.async loads and stores) are inputs it would fault on
  if (H <= 0 || HV % H) return (int)hipErrorInvalidValue;
  auto mis = [](const void* p, uintptr_t a) { return !p || (reinterpret_cast<uintptr_t>(p) & (a - 1)); };
  if (mis(q, 16) || mis(k, 16) || mis(v, 16) || mis(A, 16) || mis(o, 16) || mis(beta, 2) || mis(g, 4) || mis(cu, 8))
    return (int)hipErrorInvalidValue;
  // the norm epilogue's 8-byte accesses of out, z and the norm weight (uint2, norm_v3:282, 360, 389)
  if (NORM && (mis(na.f2s, 4) || mis(na.z, 8) || mis(na.nw, 8) || (na.ZS & 3))) return (int)hipErrorInvalidValue;
  const long long nwg = (long long)N * HV;
  if (nwg > INT32_MAX) return (int)hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((howu_kernel<DENSE, NORM>), dim3((unsigned)nwg), dim3(HW_THREADS), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                     static_cast<const uint16_t*>(v), static_cast<const uint16_t*>(beta),
                     static_cast<const uint16_t*>(A), static_cast<const float*>(g), static_cast<uint16_t*>(o),
                     static_cast<const int64_t*>(cu), scale, N, H, HV, na);
  return (int)hipGetLastError();
}

}  // namespace
}  // namespace reax

extern "C" int howu3_dense(const void* q, const void* k, const void* v, const void* beta, const void* A, const void* g,
                           void* o, const void* cu, float scale, int N, int H, int HV, void* stream) {
  return reax::launch_howu<true>(q, k, v, beta, A, g, o, cu, scale, N, H, HV, stream);
}
extern "C" int howu3_skip(const void* q, const void* k, const void* v, const void* beta, const void* A, const void* g,
                          void* o, const void* cu, float scale, int N, int H, int HV, void* stream) {
  return reax::launch_howu<false>(q, k, v, beta, A, g, o, cu, scale, N, H, HV, stream);
}
extern "C" int reax_howu(const void* q, const void* k, const void* v, const void* beta, const void* A, const void* g,
                         void* o, const void* cu, float scale, int N, int H, int HV, void* stream) {
  return reax::launch_howu<false>(q, k, v, beta, A, g, o, cu, scale, N, H, HV, stream);
}
extern "C" int reax_howu_norm(const void* q, const void* k, const void* v, const void* beta, const void* A,
                              const void* g, void* out, const void* cu, float scale, int N, int H, int HV, void* stream,
                              const void* f2s, const void* z, long long ZS, const void* nw, float eps, float factor) {
  const reax::NormArgs na{static_cast<const int*>(f2s), static_cast<const uint16_t*>(z), ZS,
                          static_cast<const uint16_t*>(nw), eps, factor};
  return reax::launch_howu<false, true>(q, k, v, beta, A, g, out, cu, scale, N, H, HV, stream, na);
}
// The kernel's LDS bytes (the reference returns its shared-memory size, howu:372).
extern "C" int howu3_smem(void) { return (int)sizeof(reax::HowuLds); }
