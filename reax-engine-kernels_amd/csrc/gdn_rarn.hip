// Reduce-add RMSNorm for gfx950: h = bf16(res + bf16(sum of S bf16 partials)), out = bf16(h * r * (1 + w)) with
// r = 1 / sqrt(factor * sum(h^2) + eps), rows of D = 2560 = 20 chunks of 128 columns. Replaces reax_rarn,
// libreax_howu/reax_rarn_final.cu:98-106 (kernel rarn2_kernel, reax_rarn_final.cu:19-90).
//
// Results follow the reference's rounding exactly except r (below):
//   - partial sum per element in fp32, partials in order 0..S-1; SERIAL rounds to bf16 after every add, otherwise
//     once at the end (rarn_final.cu:47-54); h = bf16(res + d) (rarn_final.cu:55);
//   - sum of squares: one fp32 accumulator per column c of a 128-column chunk, adding h^2 (rounded product) over the
//     chunks k = 0..19 in order (rarn_final.cu:57-58); the 128 accumulators then combine as slot sums
//     ((a[4m] + a[4m+1]) + a[4m+2]) + a[4m+3] for the 32 slots m (rarn_final.cu:63-66) and a halving tree
//     t(m) = s(m) + s(m+16), then + 8, + 4, + 2, + 1 (rarn_final.cu:67-78);
//   - r = 1 / sqrt(tot * factor + eps) with the multiply and the add rounded separately (rarn_final.cu:82). The
//     reference takes CUDA's approximate rsqrtf here; this build computes the reciprocal square root in double
//     precision and rounds it to fp32 (a value within an ulp of the reference's);
//   - out = bf16((h * r) * (1 + w)), every operation rounded (rarn_final.cu:86-87).
//
// Layout for MI355X: a row is 5 KB of bf16 per tensor; 16 lanes cover a 128-column chunk with one 16-byte access
// each, so a wavefront streams 4 rows at a time with full 64-byte segments and the loads of 4 chunks of every
// partial in flight; the per-column accumulators of a row meet in LDS for the fixed-order reduction. Rows whose
// buffers are only 4-byte aligned (the reference's own precondition) take a 2-column-per-lane form of the same
// kernel. The partials and the residual are read exactly once, with the nontemporal hint; the second pass reads h
// back from h_out, which this workgroup has just written (L2 hits), instead of holding 20 chunks in registers.
#include <hip/hip_runtime.h>
#include <stdint.h>

#pragma GCC visibility push(default)
#include "libreax_howu.h"
#pragma GCC visibility pop

#include "fmha_common.h"

namespace reax {
namespace {

constexpr int RARN_D = 2560, RARN_CH = RARN_D / 128;  // 20 chunks of 128 columns
constexpr int RARN_THREADS = 256;

__device__ __forceinline__ float bfr(float x) { return bf16lo(pack_bf16x2(x, 0.f)); }

template <int VEC>
struct Vec;
template <>
struct Vec<8> {
  typedef u32x4_t T;  // 8 bf16
};
template <>
struct Vec<2> {
  typedef uint32_t T;  // 2 bf16
};

template <int VEC>
__device__ __forceinline__ float elem(const typename Vec<VEC>::T& x, int e) {
  if constexpr (VEC == 8) {
    return (e & 1) ? bf16hi(x[e >> 1]) : bf16lo(x[e >> 1]);
  } else {
    return (e & 1) ? bf16hi(x) : bf16lo(x);
  }
}
template <int VEC>
__device__ __forceinline__ typename Vec<VEC>::T load_nt(const uint16_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const typename Vec<VEC>::T*>(p));
}
template <int VEC>
__device__ __forceinline__ typename Vec<VEC>::T load_plain(const uint16_t* p) {
  return *reinterpret_cast<const typename Vec<VEC>::T*>(p);
}

// VEC columns per lane and chunk: 128 / VEC lanes per row, 64 * VEC / 128 rows per wavefront.
template <int S, bool SERIAL, int VEC>
__global__ void __launch_bounds__(RARN_THREADS) rarn_kernel(const uint16_t* __restrict__ part, long long pstride,
                                                            const uint16_t* __restrict__ res,
                                                            const uint16_t* __restrict__ w, uint16_t* __restrict__ h_out,
                                                            uint16_t* __restrict__ out, int n, float eps, float factor) {
  constexpr int LPR = 128 / VEC;             // lanes per row
  constexpr int RPW = 64 / LPR;              // rows per wavefront
  constexpr int RPB = RPW * (RARN_THREADS / 64);  // rows per workgroup
  constexpr int NW = VEC / 2;                // packed bf16 pairs per lane and chunk
  constexpr int BATCH = S <= 4 ? 4 : 2;      // chunks whose loads are in flight together (registers: 2 waves/SIMD)
  static_assert(RARN_CH % BATCH == 0, "whole batches");
  __shared__ float red[RPB][128];
  __shared__ float rr[RPB];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int rl = wv * RPW + lane / LPR;  // row within the workgroup
  const int j = lane % LPR;              // columns VEC*j .. VEC*j + VEC-1 of every chunk
  const long long row = (long long)blockIdx.x * RPB + rl;
  const bool live = row < n;
  const long long ro = (live ? row : 0) * RARN_D + VEC * j;

  float acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.f;

  // pass 1: h, its squares, h_out (one batch of chunks at a time keeps the registers of 2 wavefronts per SIMD)
#pragma unroll 1
  for (int k0 = 0; k0 < RARN_CH; k0 += BATCH) {
    typename Vec<VEC>::T p[BATCH][S], rv[BATCH];
#pragma unroll
    for (int c = 0; c < BATCH; ++c) {
      const long long off = ro + 128 * (k0 + c);
#pragma unroll
      for (int s = 0; s < S; ++s) p[c][s] = load_nt<VEC>(part + s * pstride + off);
      rv[c] = load_nt<VEC>(res + off);
    }
#pragma unroll
    for (int c = 0; c < BATCH; ++c) {
      float h[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        float d = elem<VEC>(p[c][0], e);
#pragma unroll
        for (int s = 1; s < S; ++s) {
          d = d + elem<VEC>(p[c][s], e);
          if (SERIAL) d = bfr(d);
        }
        d = bfr(d);
        h[e] = bfr(elem<VEC>(rv[c], e) + d);
        acc[e] = acc[e] + h[e] * h[e];
      }
      uint32_t hp[NW];
#pragma unroll
      for (int q = 0; q < NW; ++q) hp[q] = pack_bf16x2(h[2 * q], h[2 * q + 1]);
      if (live) {
        uint16_t* dst = h_out + ro + 128 * (k0 + c);
        if constexpr (VEC == 8)
          *reinterpret_cast<u32x4_t*>(dst) = u32x4_t{hp[0], hp[1], hp[2], hp[3]};
        else
          *reinterpret_cast<uint32_t*>(dst) = hp[0];
      }
    }
  }

  // ---- fixed-order reduction of the 128 column accumulators of each row
#pragma unroll
  for (int e = 0; e < VEC; ++e) red[rl][VEC * j + e] = acc[e];
  __syncthreads();
  if (tid < RPB * 16) {
    // 16 lanes per row: lane m16 forms the slot sums of slots 2 m16 and 2 m16 + 1 (columns 8 m16 .. 8 m16 + 7)
    const int rrow = tid >> 4, m16 = tid & 15;
    const float* a = &red[rrow][8 * m16];
    float s0 = ((a[0] + a[1]) + a[2]) + a[3];
    float s1 = ((a[4] + a[5]) + a[6]) + a[7];
    // halving tree over the 32 slots (slot 2 m16 + b sits in lane m16, element b): + 16 slots = + 8 lanes, ...
    // + 2 slots = + 1 lane, then the last step adds the lane's two slots
#pragma unroll
    for (int d = 8; d >= 1; d >>= 1) {
      const float o0 = __shfl_down(s0, d, 16), o1 = __shfl_down(s1, d, 16);
      s0 = s0 + o0;
      s1 = s1 + o1;
    }
    if (m16 == 0) {
      const float tot = s0 + s1;
      const float x = tot * factor + eps;
      rr[rrow] = (float)(1.0 / sqrt((double)x));
    }
  }
  __syncthreads();  // also orders this lane's h_out stores before its reads below
  if (!live) return;
  const float r = rr[rl];
  // pass 2: out from h, read back from h_out (this lane's own stores, still in L2)
#pragma unroll 4
  for (int k = 0; k < RARN_CH; ++k) {
    const typename Vec<VEC>::T wv2 = load_plain<VEC>(w + 128 * k + VEC * j);
    const typename Vec<VEC>::T hv = load_plain<VEC>(h_out + ro + 128 * k);
    uint32_t o[NW];
#pragma unroll
    for (int q = 0; q < NW; ++q) {
      const float h0 = elem<VEC>(hv, 2 * q), h1 = elem<VEC>(hv, 2 * q + 1);
      const float o0 = (h0 * r) * (1.f + elem<VEC>(wv2, 2 * q));
      const float o1 = (h1 * r) * (1.f + elem<VEC>(wv2, 2 * q + 1));
      o[q] = pack_bf16x2(o0, o1);
    }
    uint16_t* dst = out + ro + 128 * k;
    if constexpr (VEC == 8)
      *reinterpret_cast<u32x4_t*>(dst) = u32x4_t{o[0], o[1], o[2], o[3]};
    else
      *reinterpret_cast<uint32_t*>(dst) = o[0];
  }
}

template <int S, bool SERIAL, int VEC>
int launch_rarn(const void* part, long long ps, const void* res, const void* w, void* h, void* o, int n, float eps,
                float f, hipStream_t st) {
  constexpr int RPB = (64 * VEC / 128) * (RARN_THREADS / 64);
  const long long nwg = ((long long)n + RPB - 1) / RPB;
  hipLaunchKernelGGL((rarn_kernel<S, SERIAL, VEC>), dim3((unsigned)nwg), dim3(RARN_THREADS), 0, st,
                     static_cast<const uint16_t*>(part), ps, static_cast<const uint16_t*>(res),
                     static_cast<const uint16_t*>(w), static_cast<uint16_t*>(h), static_cast<uint16_t*>(o), n, eps, f);
  return (int)hipGetLastError();
}

template <int S>
int launch_rarn_s(bool serial, bool vec8, const void* part, long long ps, const void* res, const void* w, void* h,
                  void* o, int n, float eps, float f, hipStream_t st) {
  if (vec8)
    return serial ? launch_rarn<S, true, 8>(part, ps, res, w, h, o, n, eps, f, st)
                  : launch_rarn<S, false, 8>(part, ps, res, w, h, o, n, eps, f, st);
  return serial ? launch_rarn<S, true, 2>(part, ps, res, w, h, o, n, eps, f, st)
                : launch_rarn<S, false, 2>(part, ps, res, w, h, o, n, eps, f, st);
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace
}  // namespace reax

extern "C" int reax_rarn(const void* part, int S, int serial, long long pstride, const void* res, const void* w,
                         void* h_out, void* out, int n, int D, float eps, float factor, void* stream) {
  using namespace reax;
  // argument checks in the reference's order (rarn_final.cu:100, 104): n <= 0 is a no-op, then D, then S
  if (D != RARN_D || n <= 0) return n <= 0 ? 0 : -1;
  if (S < 2 || S > 8) return -2;
  // inputs the reference would fault on: missing buffers, or rows not 4-byte aligned (its 4-byte accesses)
  if (!part || !res || !w || !h_out || !out) return (int)hipErrorInvalidValue;
  if (!aligned(part, 4) || !aligned(res, 4) || !aligned(w, 4) || !aligned(h_out, 4) || !aligned(out, 4) ||
      (pstride & 1))
    return (int)hipErrorInvalidValue;
  const bool vec8 = aligned(part, 16) && aligned(res, 16) && aligned(w, 16) && aligned(h_out, 16) &&
                    aligned(out, 16) && (pstride & 7) == 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool ser = serial != 0;
  switch (S) {
    case 2: return launch_rarn_s<2>(ser, vec8, part, pstride, res, w, h_out, out, n, eps, factor, st);
    case 3: return launch_rarn_s<3>(ser, vec8, part, pstride, res, w, h_out, out, n, eps, factor, st);
    case 4: return launch_rarn_s<4>(ser, vec8, part, pstride, res, w, h_out, out, n, eps, factor, st);
    case 5: return launch_rarn_s<5>(ser, vec8, part, pstride, res, w, h_out, out, n, eps, factor, st);
    case 6: return launch_rarn_s<6>(ser, vec8, part, pstride, res, w, h_out, out, n, eps, factor, st);
    case 7: return launch_rarn_s<7>(ser, vec8, part, pstride, res, w, h_out, out, n, eps, factor, st);
    default: return launch_rarn_s<8>(ser, vec8, part, pstride, res, w, h_out, out, n, eps, factor, st);
  }
}
