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
// Layout for MI355X: one workgroup of 4 wavefronts per (sequence, value head), as the reference's one CTA; every
// product is a v_mfma_f32_32x32x16_bf16 sequence over LDS operands (A operands row-major, B operands stored
// transposed so that both fragments are one 16-byte read per lane; rows XOR-swizzled in 16-byte units against bank
// conflicts). The state lives in the accumulators of the wavefronts (32 k-dims each, 4 tiles of 32 x 32) and its
// bf16 copy in LDS for the next chunk's products.
#include <hip/hip_runtime.h>
#include <stdint.h>

#pragma GCC visibility push(default)
#include "libreax_howu.h"
#pragma GCC visibility pop

#include "fmha_common.h"

namespace reax {
namespace {

constexpr int HW_BT = 64, HW_D = 128, HW_THREADS = 256;

// element (r, c) of a row-major bf16 matrix W columns wide, 16-byte units XOR-swizzled by the row. Rows of 64
// (128 bytes, two per 256-byte line of the 64 banks) also mix row / 8 into the XOR: fragment reads of 16
// consecutive rows then use 16 distinct bank groups, and the transposed 2-byte stores of 16 rows 8 apart (the
// staging of k^T, vb^T, kb^T) spread over 8 of them instead of one.
template <int W>
__device__ __forceinline__ int sw(int r, int c) {
  const int f = W == 64 ? (r ^ (r >> 3)) & 7 : r & (W / 8 - 1);
  return r * W + (((c >> 3) ^ f) << 3) + (c & 7);
}

struct HowuLds {
  uint16_t q[HW_BT * HW_D];    // [t][d]
  uint16_t k[HW_BT * HW_D];    // [s][d]: B^T of q k^T
  uint16_t kt[HW_D * HW_BT];   // [d][t]: A of k^T vdec
  uint16_t a[HW_BT * HW_BT];   // [t][s]
  uint16_t vbt[HW_D * HW_BT];  // [c][s]: B^T of A vb; then vn^T
  uint16_t kbt[HW_D * HW_BT];  // [c][s]: B^T of A kb; then vdec^T
  uint16_t wb[HW_BT * HW_D];   // [t][d]
  uint16_t hst[HW_D * HW_D];   // [c][d]: bf16(h)^T
  uint16_t aq[HW_BT * HW_BT];  // [t][s]
  float g[HW_BT], eg[HW_BT], beta[HW_BT], da[HW_BT];
};

__device__ __forceinline__ uint16_t bf16_bits(float x) { return (uint16_t)(pack_bf16x2(x, 0.f) & 0xffffu); }
__device__ __forceinline__ float bf16_val(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// acc += A[m0.., k0..k0+16*KS) . B[k0.., n0..] with A row-major (AW wide) and B stored transposed (BW wide)
template <int KS, int AW, int BW>
__device__ __forceinline__ void mm(f32x16_t& acc, const uint16_t* A, int m0, const uint16_t* BT, int n0, int k0,
                                   int lane) {
  const int r = lane & 31, kh = 8 * (lane >> 5);
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const int kc = k0 + 16 * s + kh;
    const bf16x8_t a = as_bf16x8(*reinterpret_cast<const u32x4_t*>(A + sw<AW>(m0 + r, kc)));
    const bf16x8_t b = as_bf16x8(*reinterpret_cast<const u32x4_t*>(BT + sw<BW>(n0 + r, kc)));
    acc = mfma32(a, b, acc);
  }
}
// row within a 32 x 32 accumulator tile of element v of this lane (the column is lane & 31)
__device__ __forceinline__ int trow(int v, int lane) { return 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3); }

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
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, jc = lane & 31;
  const int i_n = NSEQ - 1 - (int)(blockIdx.x / HV), hv = (int)(blockIdx.x % HV), kh = hv / (HV / H);
  const long long bos = cu[i_n];
  const int T = (int)(cu[i_n + 1] - bos);
  // 64 x 128 products: wavefront wv owns rows 32 (wv >> 1).., columns 64 (wv & 1) + 32 tt (tt = 0, 1)
  const int om0 = 32 * (wv >> 1), on0 = 64 * (wv & 1);
  // the state: k-dims 32 wv.., v-dims 32 tt (tt = 0..3)
  f32x16_t h[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int e = 0; e < 16; ++e) h[tt][e] = 0.f;

  for (int t0 = 0, it = 0; t0 < T; t0 += HW_BT, ++it) {
    const int nv = min(HW_BT, T - t0);
    // ---- stage the chunk: q, k (and k^T), A (lower block triangle unless DENSE), g, beta, then vb^T, kb^T
    if (tid < HW_BT) {
      const bool ok = tid < nv;
      const long long row = (bos + t0 + tid) * HV + hv;
      const float gg = ok ? g[row] : 0.f;
      S.g[tid] = gg;
      S.eg[tid] = fast_exp2(gg);
      S.beta[tid] = ok ? bf16_val(beta[row]) : 0.f;
    }
    for (int i = tid; i < HW_BT * (HW_D / 8); i += HW_THREADS) {
      const int t = i >> 4, c8 = (i & 15) * 8;
      u32x4_t qw = {0u, 0u, 0u, 0u}, kw = {0u, 0u, 0u, 0u};
      if (t < nv) {
        const long long ro = ((bos + t0 + t) * H + kh) * HW_D + c8;
        qw = *reinterpret_cast<const u32x4_t*>(q + ro);
        kw = *reinterpret_cast<const u32x4_t*>(k + ro);
      }
      *reinterpret_cast<u32x4_t*>(S.q + sw<HW_D>(t, c8)) = qw;
      *reinterpret_cast<u32x4_t*>(S.k + sw<HW_D>(t, c8)) = kw;
#pragma unroll
      for (int e = 0; e < 8; ++e) S.kt[sw<HW_BT>(c8 + e, t)] = (uint16_t)(kw[e >> 1] >> (16 * (e & 1)));
    }
    for (int i = tid; i < HW_BT * (HW_BT / 8); i += HW_THREADS) {
      const int t = i >> 3, c8 = (i & 7) * 8;
      u32x4_t aw = {0u, 0u, 0u, 0u};
      if (t < nv && (DENSE || (c8 >> 4) <= (t >> 4)))
        aw = *reinterpret_cast<const u32x4_t*>(Ag + ((bos + t0 + t) * HV + hv) * HW_BT + c8);
      *reinterpret_cast<u32x4_t*>(S.a + sw<HW_BT>(t, c8)) = aw;
    }
    __syncthreads();
    for (int i = tid; i < HW_BT * (HW_D / 8); i += HW_THREADS) {
      const int t = i >> 4, c8 = (i & 15) * 8;
      u32x4_t vw = {0u, 0u, 0u, 0u};
      if (t < nv) vw = *reinterpret_cast<const u32x4_t*>(v + ((bos + t0 + t) * HV + hv) * HW_D + c8);
      const u32x4_t kw = *reinterpret_cast<const u32x4_t*>(S.k + sw<HW_D>(t, c8));
      const float b = S.beta[t], e = S.eg[t];
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        const float vv = (x & 1) ? bf16hi(vw[x >> 1]) : bf16lo(vw[x >> 1]);
        const float kk = (x & 1) ? bf16hi(kw[x >> 1]) : bf16lo(kw[x >> 1]);
        S.vbt[sw<HW_BT>(c8 + x, t)] = bf16_bits(vv * b);
        S.kbt[sw<HW_BT>(c8 + x, t)] = bf16_bits(bf16_val(bf16_bits(kk * b)) * e);
      }
    }
    __syncthreads();

    // ---- u = A vb (kept as bf16 values), wb = bf16(A kb) -> LDS, AQ -> LDS
    float ub[2][16];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      f32x16_t cu_ = {}, cw = {};
      mm<4, HW_BT, HW_BT>(cu_, S.a, om0, S.vbt, on0 + 32 * tt, 0, lane);
      mm<4, HW_BT, HW_BT>(cw, S.a, om0, S.kbt, on0 + 32 * tt, 0, lane);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        ub[tt][e] = bf16_val(bf16_bits(cu_[e]));
        S.wb[sw<HW_D>(om0 + trow(e, lane), on0 + 32 * tt + jc)] = bf16_bits(cw[e]);
      }
    }
    {
      const int am0 = 32 * (wv >> 1), an0 = 32 * (wv & 1);
      f32x16_t c = {};
      if (an0 <= am0) mm<8, HW_D, HW_D>(c, S.q, am0, S.k, an0, 0, lane);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int t = am0 + trow(e, lane), s = an0 + jc;
        float y = 0.f;
        if (s <= t && t < nv) y = c[e] * fast_exp2(S.g[t] - S.g[s]);
        S.aq[sw<HW_BT>(t, s)] = bf16_bits(y);
      }
    }
    const float glast = S.g[nv - 1];
    if (tid < HW_BT) S.da[tid] = tid < nv ? fast_exp2(glast - S.g[tid]) : 0.f;
    __syncthreads();

    // ---- vw = wb bf16(h), oi = q bf16(h); vn, vdec (transposed into the vb^T / kb^T buffers)
    float oi[2][16];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      f32x16_t cvw = {}, coi = {};
      if (it > 0) {
        mm<8, HW_D, HW_D>(cvw, S.wb, om0, S.hst, on0 + 32 * tt, 0, lane);
        mm<8, HW_D, HW_D>(coi, S.q, om0, S.hst, on0 + 32 * tt, 0, lane);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        oi[tt][e] = coi[e];
        const int t = om0 + trow(e, lane), c = on0 + 32 * tt + jc;
        const float x = ub[tt][e] - cvw[e];
        S.vbt[sw<HW_BT>(c, t)] = bf16_bits(x);
        S.kbt[sw<HW_BT>(c, t)] = bf16_bits(x * S.da[t]);
      }
    }
    __syncthreads();

    // ---- o = bf16(fma(AQ vn, scale, (oi eg) scale)); h = h 2^glast + k^T vdec
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      f32x16_t ci = {};
      mm<4, HW_BT, HW_BT>(ci, S.aq, om0, S.vbt, on0 + 32 * tt, 0, lane);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int t = om0 + trow(e, lane), c = on0 + 32 * tt + jc;
        const float r = __builtin_fmaf(ci[e], scale, (oi[tt][e] * S.eg[t]) * scale);
        if (NORM)
          S.wb[sw<HW_D>(t, c)] = bf16_bits(r);  // staged for the epilogue (wb is free after vw)
        else if (t < nv)
          o[((bos + t0 + t) * HV + hv) * HW_D + c] = bf16_bits(r);
      }
    }
    const float gl = fast_exp2(glast);
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
#pragma unroll
      for (int e = 0; e < 16; ++e) h[tt][e] = h[tt][e] * gl;
      mm<4, HW_BT, HW_BT>(h[tt], S.kt, 32 * wv, S.kbt, 32 * tt, 0, lane);
    }
    __syncthreads();  // every read of this chunk's LDS is done (and the staged o rows are visible)
    if (NORM) {
      // two rows per wavefront at a time, one per 32-lane half: lane l of a half holds columns 4l .. 4l+3
      const int half = lane >> 5, l32 = lane & 31;
#pragma unroll 1
      for (int i = 0; i < HW_BT / 8; ++i) {
        const int t = 2 * (wv * (HW_BT / 8) + i) + half;
        const int R = t < nv ? na.f2s[bos + t0 + t] : -1;
        if (R < 0) continue;  // the same for the whole half
        const u32x2_t xo = *reinterpret_cast<const u32x2_t*>(S.wb + sw<HW_D>(t, 4 * l32));
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
          const float y = bf16_val(bf16_bits(x[e] * rr));
          const float y2 = bf16_val(bf16_bits(w[e] * y));
          res[e] = y2 * silu_f32(zz[e]);
        }
        *reinterpret_cast<u32x2_t*>(o + ((long long)R * HV + hv) * HW_D + 4 * l32) =
            u32x2_t{pack_bf16x2(res[0], res[1]), pack_bf16x2(res[2], res[3])};
      }
    }
    // bf16(h)^T for the next chunk: element (d, c) of the state at hst[c][d]
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
      for (int e = 0; e < 16; ++e) S.hst[sw<HW_D>(32 * tt + jc, 32 * wv + trow(e, lane))] = bf16_bits(h[tt][e]);
    // (the next chunk's staging writes other buffers; its first barrier orders these stores before their reads)
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
