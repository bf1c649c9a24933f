// Causal 4-tap conv1d + SiLU (+ L2 normalisation of the q/k heads) for gfx950. Replaces reax_conv_l2 and reax_conv_v,
// libreax_howu/reax_conv_v2.cu:164-189 (kernel conv_l2_kernel, reax_conv_v2.cu:60-150).
//
// Per token t and channel c (units of 128 channels: q heads, k heads, then v heads):
//   tap j = 0..3 reads source row src = meta[t].x - 3 + j (skipped when src < 0): row meta[t].z + src of qkv (row
//   stride SX) when src >= meta[t].y, else row meta[t].w + src of the conv cache (row stride C)   (conv_v2:88-92)
//   acc = fp32 sum over the taps in order of w[c][j] * x (each product exact, each add rounded)     (conv_v2:96-108)
//   y = bf16(acc); s = bf16(y / (1 + exp(-y)))                                                     (conv_v2:112-122)
//   q/k units: out = bf16(s * rstd), rstd = 1 / sqrt(eps + sum of s^2 over the 128 channels), the sum formed per
//   8-channel group as s1^2 + s0^2 + s2^2 + ... + s7^2 and then combined across the 16 groups by a butterfly over
//   group distance 8, 4, 2, 1 (conv_v2:123-132); rep = 2 writes each q/k head twice, side by side (conv_v2:139-142)
//   v units: out = s                                                                               (conv_v2:143-147)
// The reference evaluates exp, the square root and the reciprocal with CUDA's fast approximations (a restated
// libdevice expf, sqrt.approx, div.full); this build defines SiLU as bf16(y / fp32(1 + exp(-y))) with exp in double
// precision and an IEEE fp32 division (the reference's division is exact to its divisor), evaluated by an fp32
// fast path that provably rounds to the same bf16 value (silu_bf16), and 1/sqrt in double precision rounded to
// fp32: the fp32 values agree with the reference's to about an ulp, so a bf16 result can differ by one bf16 ulp in
// rare elements that sit on a rounding boundary.
//
// Layout for MI355X: 16 lanes cover a 128-channel unit with 16-byte accesses (8 channels per lane); a workgroup
// takes 16 neighbouring units (4 KB of each source row, read and written contiguously) through 4 tokens, each
// 16-lane group holding its unit's 4 taps x 128 weights in registers; the overlapping source rows of neighbouring
// tokens hit in cache, so HBM sees each row about once.
#include <hip/hip_runtime.h>
#include <stdint.h>

#pragma GCC visibility push(default)
#include "libreax_howu.h"
#pragma GCC visibility pop

#include "fmha_common.h"

namespace reax {
namespace {

constexpr int CONV_THREADS = 256;
constexpr int CONV_UNITS = CONV_THREADS / 16;  // 128-channel units per workgroup (one per 16-lane group)
constexpr int CONV_TOK = 4;                    // tokens per workgroup (measured: 4 and 2 beat 16 by 8%, 1 is slower)

__device__ __forceinline__ float bfr(float x) { return bf16lo(pack_bf16x2(x, 0.f)); }

// bf16(y / d) with d = 1 + exp(-y) rounded to fp32 (infinite when exp(-y) overflows it) and an IEEE fp32 division.
// Slow path: exactly that, with exp in double precision. Kept out of line: it is taken for a few elements at most.
__device__ __attribute__((noinline)) float silu_bf16_slow(float y) {
  const float d = (float)(1.0 + exp(-(double)y));
  return bfr(y / d);
}
// Fast path for |y| < 64 (y is a bf16 value, 8 significant bits): -y log2 e = a_hi + a_lo with a_hi = -y * H exact
// (H = log2 e cut to 16 significant bits, so the product needs at most 24) and a_lo = -y * (log2 e - H), |a_lo| <
// 5e-4; e = 2^a_hi (v_exp_f32, 1 ulp) * (1 + t + t^2/2) with t = a_lo ln 2 (the dropped t^3/6 is below 1e-11),
// about 2 ulp in all; then d' = 1 + e and q' = y * rcp(d') (v_rcp_f32, 1 ulp): q' lies within 9 ulp of the slow
// path's fp32 quotient q. Whenever q' is within 32 ulp of a bf16 rounding midpoint the slow path decides; otherwise
// q' and q round to the same bf16 value, so the result equals the slow path's bit for bit.
// Returns the fast result and sets ok = false when the slow path must decide instead (|y| >= 64, NaN, or q' near a
// midpoint); the caller batches those.
__device__ __forceinline__ float silu_bf16_fast(float y, bool& ok) {
  const float a_hi = y * -1.44268798828125f;
  const float a_lo = y * -7.052607543300837e-06f;
  const float t = a_lo * 0.6931471824645996f;
  const float eh = fast_exp2(a_hi);
  const float e = __builtin_fmaf(eh, __builtin_fmaf(0.5f * t, t, t), eh);
  const float q = y * __builtin_amdgcn_rcpf(1.0f + e);
  const uint32_t low = __float_as_uint(q) & 0xffffu;
  ok = (y > -64.0f && y < 64.0f) && !(low > 0x8000u - 32u && low < 0x8000u + 32u);
  return bfr(q);
}

template <int REP, bool SKIP_V>
__global__ void __launch_bounds__(CONV_THREADS) conv_kernel(const uint16_t* __restrict__ qkv, long long SX,
                                                            const uint16_t* __restrict__ cache, int C,
                                                            const int* __restrict__ meta, const uint16_t* __restrict__ w,
                                                            uint16_t* __restrict__ q, uint16_t* __restrict__ k,
                                                            uint16_t* __restrict__ v, int Tf, float eps, int KD, int VD,
                                                            int u0, int n_units) {
  const int tid = threadIdx.x, grp = tid >> 4, l16 = tid & 15;
  const int u = u0 + blockIdx.y * CONV_UNITS + grp;
  if (u >= u0 + n_units) return;  // whole 16-lane groups; no barrier below
  const int c0 = u * 128 + 8 * l16;
  const int nqk = 2 * KD / 128;
  const bool is_qk = u < nqk;

  // weights of this lane's 8 channels: w[c][0..3] for c = c0 .. c0 + 7, one 8-byte access per channel
  float wt[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const u32x2_t x = *reinterpret_cast<const u32x2_t*>(w + (long long)(c0 + i) * 4);
    wt[i][0] = bf16lo(x[0]);
    wt[i][1] = bf16hi(x[0]);
    wt[i][2] = bf16lo(x[1]);
    wt[i][3] = bf16hi(x[1]);
  }

#pragma unroll 4
  for (int i = 0; i < CONV_TOK; ++i) {
    const int t = blockIdx.x * CONV_TOK + i;
    const bool live = t < Tf;
    const int4 m = live ? *reinterpret_cast<const int4*>(meta + (long long)t * 4) : make_int4(-100, 0, 0, 0);
    // every tap loads (a skipped tap, src < 0, reads qkv's first row instead and is not accumulated), so the
    // loads of several tokens can be in flight together
    u32x4_t xv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int src = m.x - 3 + j;
      const uint16_t* rp = src < 0 ? qkv : src >= m.y ? qkv + (long long)(m.z + src) * SX : cache + (long long)(m.w + src) * C;
      xv[j] = *reinterpret_cast<const u32x4_t*>(rp + c0);
    }
    float acc[8];
    if (m.x >= 3) {  // all four taps (the same for the whole workgroup: one token)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        acc[i] = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i] = __builtin_fmaf(wt[i][j], (i & 1) ? bf16hi(xv[j][i >> 1]) : bf16lo(xv[j][i >> 1]), acc[i]);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        acc[i] = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float f = __builtin_fmaf(wt[i][j], (i & 1) ? bf16hi(xv[j][i >> 1]) : bf16lo(xv[j][i >> 1]), acc[i]);
          acc[i] = m.x - 3 + j >= 0 ? f : acc[i];
        }
      }
    }
    float s[8], y[8];
    bool all_ok = true;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      y[i] = bfr(acc[i]);
      bool ok;
      s[i] = silu_bf16_fast(y[i], ok);
      all_ok &= ok;
    }
    // the few elements the fast path cannot decide, once per token for the whole lane
    if (__builtin_expect(!all_ok, 0)) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        bool ok;
        silu_bf16_fast(y[i], ok);
        if (!ok) s[i] = silu_bf16_slow(y[i]);
      }
    }
    if (is_qk) {
      float sum = s[1] * s[1];
      sum = __builtin_fmaf(s[0], s[0], sum);
#pragma unroll
      for (int i = 2; i < 8; ++i) sum = __builtin_fmaf(s[i], s[i], sum);
      // butterfly over the 16 lanes of the unit: every lane ends with the same total
#pragma unroll
      for (int d = 8; d >= 1; d >>= 1) sum = sum + __shfl_xor(sum, d, 16);
      const float rstd = (float)(1.0 / sqrt((double)(eps + sum)));
      if (!live) continue;
      u32x4_t ov;
#pragma unroll
      for (int p = 0; p < 4; ++p) ov[p] = pack_bf16x2(rstd * s[2 * p], rstd * s[2 * p + 1]);
      const int nh = REP * KD / 128, hq = u % (KD / 128);
      uint16_t* dst = (u < KD / 128 ? q : k) + (long long)t * (nh * 128) + REP * hq * 128 + 8 * l16;
      *reinterpret_cast<u32x4_t*>(dst) = ov;
      if (REP == 2) *reinterpret_cast<u32x4_t*>(dst + 128) = ov;
    } else if (!SKIP_V) {
      if (!live) continue;
      u32x4_t ov;
#pragma unroll
      for (int p = 0; p < 4; ++p) ov[p] = pack_bf16x2(s[2 * p], s[2 * p + 1]);
      *reinterpret_cast<u32x4_t*>(v + (long long)t * VD + (c0 - 2 * KD)) = ov;
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int launch_conv(const void* qkv, long long SX, const void* cache, int C, const void* meta, const void* w, void* q,
                void* k, void* v, int Tf, float eps, int KD, int VD, int rep, int skip_v, int u0, int units,
                hipStream_t st) {
  if (units <= 0) return 0;
  const unsigned gx = (unsigned)((Tf + CONV_TOK - 1) / CONV_TOK);
  const dim3 grid(gx, (unsigned)((units + CONV_UNITS - 1) / CONV_UNITS));
  auto* a = static_cast<const uint16_t*>(qkv);
  auto* cc = static_cast<const uint16_t*>(cache);
  auto* mt = static_cast<const int*>(meta);
  auto* ww = static_cast<const uint16_t*>(w);
  auto *qq = static_cast<uint16_t*>(q), *kk = static_cast<uint16_t*>(k), *vv = static_cast<uint16_t*>(v);
  if (rep == 1 && !skip_v)
    hipLaunchKernelGGL((conv_kernel<1, false>), grid, dim3(CONV_THREADS), 0, st, a, SX, cc, C, mt, ww, qq, kk, vv, Tf, eps, KD, VD, u0, units);
  else if (rep == 1)
    hipLaunchKernelGGL((conv_kernel<1, true>), grid, dim3(CONV_THREADS), 0, st, a, SX, cc, C, mt, ww, qq, kk, vv, Tf, eps, KD, VD, u0, units);
  else if (!skip_v)
    hipLaunchKernelGGL((conv_kernel<2, false>), grid, dim3(CONV_THREADS), 0, st, a, SX, cc, C, mt, ww, qq, kk, vv, Tf, eps, KD, VD, u0, units);
  else
    hipLaunchKernelGGL((conv_kernel<2, true>), grid, dim3(CONV_THREADS), 0, st, a, SX, cc, C, mt, ww, qq, kk, vv, Tf, eps, KD, VD, u0, units);
  return (int)hipGetLastError();
}

// Shapes and buffers the kernel relies on (the reference faults, or reads out of its buffers, without them):
// whole 128-channel heads (KD < 128 divides by zero there, conv_v2:139), 16-byte aligned rows and meta entries
// (its uint4 / int4 accesses, conv_v2:75, 91, 141, 147) and 8-byte aligned weights (uint2, conv_v2:80). This build
// also reads qkv's first row for taps before position 0, so qkv must hold at least one row (it holds the Tf new
// tokens in the engine's use).
bool conv_args_ok(const void* qkv, long long SX, const void* cache, int C, const void* meta, const void* w, int KD,
                  int VD) {
  if (!qkv || !cache || !meta || !w) return false;
  if (KD <= 0 || KD % 128 || VD < 0 || VD % 128) return false;
  if (!aligned16(qkv) || !aligned16(cache) || !aligned16(meta) || (reinterpret_cast<uintptr_t>(w) & 7u) || (SX & 7) ||
      (C & 7))
    return false;
  return true;
}

}  // namespace
}  // namespace reax

extern "C" int reax_conv_l2(const void* qkv, long long SX, const void* cache, int C, const void* meta, const void* w,
                            void* q, void* k, void* v, int Tf, float eps, int KD, int VD, int rep, int skip_v, int RT,
                            void* stream) {
  using namespace reax;
  if (Tf <= 0) return 0;                                     // conv_v2:166
  if (RT != 8 && RT != 16 && RT != 32) return -1;            // conv_v2:173-177 (a tiling choice there; checked only)
  if (!conv_args_ok(qkv, SX, cache, C, meta, w, KD, VD)) return (int)hipErrorInvalidValue;
  if (!q || !k || !aligned16(q) || !aligned16(k) || (!skip_v && (!v || !aligned16(v)))) return (int)hipErrorInvalidValue;
  const int units = 2 * KD / 128 + (skip_v ? 0 : VD / 128);
  // rep == 1: one copy of each q/k head; any other value: two (conv_v2:158-161)
  return launch_conv(qkv, SX, cache, C, meta, w, q, k, v, Tf, eps, KD, VD, rep == 1 ? 1 : 2, skip_v != 0, 0, units,
                     static_cast<hipStream_t>(stream));
}

extern "C" int reax_conv_v(const void* qkv, long long SX, const void* cache, int C, const void* meta, const void* w,
                           void* v, int Tf, int KD, int VD, void* stream) {
  using namespace reax;
  if (Tf <= 0) return 0;  // conv_v2:185
  if (!conv_args_ok(qkv, SX, cache, C, meta, w, KD, VD) || !v || !aligned16(v)) return (int)hipErrorInvalidValue;
  // the value units only (conv_v2:186-187): units 2*KD/128 .. 2*KD/128 + VD/128 - 1, no q/k outputs
  return launch_conv(qkv, SX, cache, C, meta, w, nullptr, nullptr, v, Tf, 1e-6f, KD, VD, 1, 0, 2 * KD / 128,
                     VD / 128, static_cast<hipStream_t>(stream));
}
