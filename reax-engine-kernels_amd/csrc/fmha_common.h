// Shared device helpers and the parameter block of the REAX FMHA kernels for gfx950 (CDNA4).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace reax {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// Mask modes of the forward kernel.
//   QPOS   : row r of batch b sees keys 0..qpos[b*qpBs + r/G]          (reax_fmha_v8.cu:9-10, 147-148)
//   BIAS   : every key visible, additive bf16 bias per (row, key)       (reax_fmha_v8.cu:11, 150-152, 279-280)
//   VARLEN : packed sequences (cu_seqlens); row r of sequence b sees its own keys 0..r/G (causal)
enum MaskMode : int { MODE_QPOS = 0, MODE_BIAS = 1, MODE_VARLEN = 2 };

// Everything a forward launch needs. Strides are in elements. Row r of (b, h) addresses
//   Q: q + b*qsB + h*qsH + (tok0 + r/G)*qsT + (r%G)*qsG     (tok0 = cu_seqlens[b] in VARLEN mode, else 0)
// and the same with the o*/ls* strides for O and LSE. K/V key j: k + b*ksB + h*ksH + (tok0 + j)*ksM.
struct FwdParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;  // may be null (POST mode writes outp instead)
  float* lse;   // optional
  const int* qpos;
  const uint16_t* bias;
  const int* cu_seqlens;
  long long qpBs;
  long long bsB, bsH, bsM;
  long long qsB, qsH, qsT, qsG;
  long long ksB, ksH, ksM;
  long long vsB, vsH, vsM;
  long long osB, osH, osT, osG;
  long long lsB, lsH, lsT, lsG;
  // POST epilogue (reax_fmha_qp): out[inv[b*Lq + r/G]][(h*G + r%G)*D + d] = bf16(bf16(o)*bf16(sigmoid(gate)))
  const int* inv;
  const uint16_t* qg;
  uint16_t* outp;
  long long qg_rs, out_rs;
  int Lq;
  // split-KV partials (SPLIT kernels): key split s of (b, h) covers keys [s*split_len, (s+1)*split_len);
  // ws_o[((bh*num_splits + s)*M + r)*D + d] = partial O normalised by its own row sum, ws_lse likewise.
  float* ws_o;
  float* ws_lse;
  int num_splits;
  int split_len;
  int B, H, G, M, N;
  // The drop-in entry points (reax_fmha_q / reax_fmha_qp) follow the reference's block-wide shortcut: folded rows
  // of (b, h) form blocks of 64 ([64j, 64j + 64)); when the largest raw qpos of a block's rows is exactly 0, every
  // row of the block, rows with qpos < 0 included, is stored as V[0] (reax_fmha_v8.cu:155-162, 224-235;
  // reax_fmha_v11.cu:213-220, 282-293). The extension entry points keep the per-row rule (qpos < 0 -> 0).
  int qpos0_block;
  int n_tiles;       // row tiles per (b, h)
  float scale;       // softmax scale
  float scale_log2;  // scale * log2(e)
};

__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Round-to-nearest-even fp32 -> bf16 pair packed as (lo | hi << 16): one v_cvt_pk_bf16_f32 on gfx950.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
}

// s_waitcnt immediate that waits until at most n (< 64) vector-memory loads of this wavefront are outstanding and
// leaves the export and LDS/scalar counters unconstrained (vmcnt bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8])
constexpr int vmcnt_le(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Combine a value with the one held 32 lanes away (the other half of the wavefront). v_permlane32_swap
// exchanges the upper half of its first operand with the lower half of its second; with x in both, one result
// holds the lower half's x in every lane and the other the upper half's, so max / sum of the two results give
// the two-lane reduction in every lane.
__device__ __forceinline__ float halves_max(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t x) { return __builtin_bit_cast(bf16x8_t, x); }

__device__ __forceinline__ f32x16_t mfma32(bf16x8_t a, bf16x8_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4_t mfma16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Sigmoid of a bf16 gate, rounded to bf16 (bits), correctly rounded for every one of the 65,536 inputs.
// Fast path: s = 1 / (1 + 2^(-x*log2(e))) in fp32 with v_exp_f32 / v_rcp_f32. For |x| < 64 the rounding of
// the exponent argument (|x*log2 e| < 93, half an ulp = 2^-18) bounds the relative error of s by about 45 fp32
// ulp, plus a few ulp for v_exp_f32, the add and v_rcp_f32. Whenever the fp32 result lies within 256 ulp of a
// bf16 rounding midpoint, or |x| >= 64, the value is recomputed in double precision, whose error is far below
// the distance to any midpoint; otherwise rounding the fp32 value to bf16 gives the correctly rounded result.
// Correctly rounded bf16 sigmoid of a gate whose fp32 fast path may round the wrong way (near a bf16 midpoint)
// or lose accuracy (|x| >= 64): double precision. Kept out of line: the epilogue calls it for a few gates at most,
// and inlined at each of its call sites the double-precision code would raise the register count of the whole
// kernel, main loop included.
__device__ __attribute__((noinline)) uint32_t sigmoid_bf16_slow(float x) {
  if (x != x) return 0x7fc0u;
  const double xd = (double)x;
  const double sd = xd >= 0.0 ? 1.0 / (1.0 + exp(-xd)) : exp(xd) / (1.0 + exp(xd));
  // sd is in [0, 1]: round it to the bf16 grid of its binade (8 significant bits, or the subnormal
  // spacing 2^-133 below 2^-126) with round-half-even.
  if (sd == 0.0) return 0u;
  int ex;
  const double m = frexp(sd, &ex);  // sd = m * 2^ex, m in [0.5, 1)
  double r;
  if (ex - 1 < -126) {
    r = ldexp(rint(ldexp(sd, 133)), -133);  // bf16 subnormal spacing 2^-133
  } else {
    r = ldexp(rint(ldexp(m, 8)), ex - 8);
  }
  return __float_as_uint((float)r) >> 16;
}
__device__ __forceinline__ uint32_t sigmoid_bf16_bits(uint32_t gbits) {
  const float x = __uint_as_float(gbits << 16);
  const float e = fast_exp2(x * -1.44269504088896340736f);
  const float s = __builtin_amdgcn_rcpf(1.0f + e);
  const uint32_t u = __float_as_uint(s);
  const uint32_t low = u & 0xffffu;
  const bool near_tie = (low > 0x8000u - 256u) && (low < 0x8000u + 256u);
  const bool bad = near_tie || !(x > -64.0f && x < 64.0f);
  if (__builtin_expect(bad, 0)) return sigmoid_bf16_slow(x);
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

}  // namespace reax
