// Gated-DeltaNet chunk solve for gfx950: per 64-token chunk of a sequence and per value head,
//   A = (I + M)^-1,  M[r][c] = (k_r . k_c) * 2^(g[r] - g[c]) * beta[r] for c < r (both rows of the chunk), else 0,
// stored as bf16 rows of 64 (the lower block triangle of 16 x 16 blocks: columns up to the end of the row's own
// 16-column block; later columns are left untouched). Replaces reax_kkt, libreax_howu/reax_kkt.cu:263-272 (kernel
// kkt7_kernel, reax_kkt.cu:79-261): one key head's k k^T serves its two value heads (HV = 2H, kkt:265).
//
// The reference forms k k^T with bf16 tensor-core MMAs, the decay with the approximate ex2, the 16 x 16 diagonal
// inverses by forward substitution and the off-diagonal blocks with tf32 MMAs (10-bit mantissa operands). This build
// forms k k^T on the matrix cores too (bf16 products are exact, fp32 accumulation) and the rest in fp32
// (v_exp_f32, full-precision forward substitution), so its results are at least as close to the exact inverse;
// agreement with the reference is to its own tf32/bf16 accuracy, not bit for bit.
//
// Layout: one workgroup of 256 threads per (chunk, key head), 34 KB of LDS (M packed as a triangle) so that four
// workgroups share a CU and one's solve overlaps the others' loads and products. Phase 1 stages the chunk's k (64 x 128 bf16, 16-byte units XOR-swizzled by row),
// g and beta; phase 2 forms k k^T with v_mfma_f32_32x32x16_bf16 (wavefronts 0-2: the two diagonal 32 x 32 tiles and
// the one below them) and writes M for both value heads straight from the accumulators (decay, mask and beta);
// phase 3 solves (I + M) X = I column by column (128 threads: 2 heads x 64 columns, the column in registers, M read
// by broadcast) and writes each column's bf16 entries straight to A (a wavefront's 64 lanes hold 64 adjacent
// columns of one row: 128 contiguous bytes per store).
#include <hip/hip_runtime.h>
#include <stdint.h>

#pragma GCC visibility push(default)
#include "libreax_howu.h"
#pragma GCC visibility pop

#include "fmha_common.h"

namespace reax {
namespace {

constexpr int KKT_BT = 64, KKT_K = 128, KKT_THREADS = 256;

__device__ __forceinline__ uint16_t bf16_bits(float x) { return (uint16_t)(pack_bf16x2(x, 0.f) & 0xffffu); }

// Row r of M (columns 0 .. r-1, padded to a multiple of 4 so that every row starts 16-byte aligned for the
// broadcast reads of the solve) starts at moff(r) floats: the strictly lower triangle in 2112 floats per head.
__host__ __device__ constexpr int moff(int r) {
  return r == 0 ? 0 : 4 * (2 * ((r - 1) / 4) * ((r - 1) / 4 + 1) + ((r - 1) % 4) * ((r - 1) / 4 + 1));
}
constexpr int KKT_MTRI = moff(KKT_BT);

struct KktLds {
  uint16_t k[KKT_BT * KKT_K];  // k rows, 16-byte units XOR-swizzled by row
  float m[2][KKT_MTRI];        // M of each value head, packed rows
  float g[2][KKT_BT];
  float beta[2][KKT_BT];
};

// element (r, c) of the staged k: 16 units of 8 per row, unit index XOR row % 16
__device__ __forceinline__ int ksw(int r, int c) { return r * KKT_K + ((((c >> 3) ^ (r & 15))) << 3) + (c & 7); }

__global__ void __launch_bounds__(KKT_THREADS, 4) kkt_kernel(const uint16_t* __restrict__ k, const float* __restrict__ g,
                                                             const uint16_t* __restrict__ beta, uint16_t* __restrict__ A,
                                                             const int64_t* __restrict__ cu,
                                                             const int64_t* __restrict__ cidx, int H, int HV) {
  __shared__ __align__(16) KktLds S;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int i_n = (int)cidx[2 * (long long)blockIdx.x], i_t = (int)cidx[2 * (long long)blockIdx.x + 1];
  const int kh = blockIdx.y;
  const long long bos = cu[i_n];
  const int T = (int)(cu[i_n + 1] - bos);
  const int t0 = i_t * KKT_BT;
  const int nval = min(KKT_BT, T - t0);

  // ---- phase 1: k rows (zero beyond the chunk's valid rows), g and beta of the two value heads
#pragma unroll
  for (int e = 0; e < KKT_BT * (KKT_K / 8) / KKT_THREADS; ++e) {
    const int i = tid + KKT_THREADS * e, r = i >> 4, c8 = (i & 15) * 8;
    u32x4_t w = {0u, 0u, 0u, 0u};
    if (r < nval) w = *reinterpret_cast<const u32x4_t*>(k + ((bos + t0 + r) * H + kh) * KKT_K + c8);
    *reinterpret_cast<u32x4_t*>(S.k + ksw(r, c8)) = w;
  }
  if (tid < 2 * KKT_BT) {
    const int v = tid >> 6, r = tid & 63, hv = 2 * kh + v;
    S.g[v][r] = r < nval ? g[(bos + t0 + r) * HV + hv] : 0.f;
    S.beta[v][r] = r < nval ? bf16lo(beta[(bos + t0 + r) * HV + hv]) : 0.f;
  }
  __syncthreads();

  // ---- phase 2: k k^T on the matrix cores for the tiles on and below the diagonal (wavefront 0: rows and columns
  // 0-31, 1: rows 32-63 x columns 0-31, 2: rows and columns 32-63), then M[v][r][c] = (k_r . k_c) 2^(g_r - g_c)
  // beta_r for c < r < nval, else 0 (entries on or above the diagonal are never read by the solve)
  if (wv < 3) {
    const int I = wv == 0 ? 0 : 1, J = wv == 2 ? 1 : 0;
    const int rr = lane & 31, kq = 8 * (lane >> 5);
    f32x16_t acc = {};
#pragma unroll
    for (int s = 0; s < KKT_K / 16; ++s) {
      const bf16x8_t a = as_bf16x8(*reinterpret_cast<const u32x4_t*>(S.k + ksw(32 * I + rr, 16 * s + kq)));
      const bf16x8_t b = as_bf16x8(*reinterpret_cast<const u32x4_t*>(S.k + ksw(32 * J + rr, 16 * s + kq)));
      acc = mfma32(a, b, acc);
    }
    const int c = 32 * J + rr;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int r = 32 * I + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
      if (c < r) {  // the solve reads only the strictly lower triangle
        const bool live = r < nval;
#pragma unroll
        for (int v = 0; v < 2; ++v)
          S.m[v][moff(r) + c] = live ? (acc[e] * fast_exp2(S.g[v][r] - S.g[v][c])) * S.beta[v][r] : 0.f;
      }
    }
  }
  __syncthreads();

  // ---- phase 3: (I + M) X = I by forward substitution, one column j per thread: x_j = 1, x_r = 0 for r < j,
  // x_r = -sum_{c<r} M[r][c] x_c for r > j (the terms with c < j vanish)
  if (tid < 2 * KKT_BT) {
    const int v = tid >> 6, j = tid & 63;
    const float* M = S.m[v];
    // entry (r, j) goes to A row r (stride HV * 64 elements) for r < nval and j up to the end of row r's own
    // 16-column block; later columns are left untouched
    uint16_t* dst = A + ((bos + t0) * HV + 2 * kh + v) * KKT_BT + j;
    const long long rs = (long long)HV * KKT_BT;
    float x[KKT_BT];
#pragma unroll
    for (int r = 0; r < KKT_BT; ++r) {
      float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
      for (int c = 0; c + 3 < r; c += 4) {
        const f32x4_t mr = *reinterpret_cast<const f32x4_t*>(&M[moff(r) + c]);
        s0 = __builtin_fmaf(mr[0], x[c], s0);
        s1 = __builtin_fmaf(mr[1], x[c + 1], s1);
        s2 = __builtin_fmaf(mr[2], x[c + 2], s2);
        s3 = __builtin_fmaf(mr[3], x[c + 3], s3);
      }
#pragma unroll
      for (int c = r & ~3; c < r; ++c) s0 = __builtin_fmaf(M[moff(r) + c], x[c], s0);
      const float s = (s0 + s1) + (s2 + s3);
      x[r] = r < j ? 0.f : r == j ? 1.f : 0.f - s;  // 0 - s: an exact zero is stored as +0
      if (r < nval && j < 16 * (r / 16 + 1)) dst[r * rs] = bf16_bits(x[r]);
    }
  }
}

}  // namespace
}  // namespace reax

extern "C" int reax_kkt(const void* k, const void* g, const void* beta, void* A, const void* cu, const void* cidx,
                        int NT, int H, int HV, void* stream) {
  using namespace reax;
  if (HV != 2 * H) return -1;  // kkt:265
  // an empty grid: the reference's launch fails with the invalid-configuration error
  if (NT <= 0 || H <= 0) return (int)hipErrorInvalidConfiguration;
  // inputs the reference would fault on: missing buffers, k rows not 16-byte aligned (uint4 loads, kkt:95), A not
  // 4-byte aligned (bf16 pairs, kkt:197-198), cu / cidx not 8-byte aligned (int64)
  if (!k || !g || !beta || !A || !cu || !cidx || (reinterpret_cast<uintptr_t>(k) & 15u) ||
      (reinterpret_cast<uintptr_t>(A) & 3u) || (reinterpret_cast<uintptr_t>(cu) & 7u) ||
      (reinterpret_cast<uintptr_t>(cidx) & 7u))
    return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(kkt_kernel, dim3((unsigned)NT, (unsigned)H), dim3(KKT_THREADS), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(k), static_cast<const float*>(g),
                     static_cast<const uint16_t*>(beta), static_cast<uint16_t*>(A), static_cast<const int64_t*>(cu),
                     static_cast<const int64_t*>(cidx), H, HV);
  return (int)hipGetLastError();
}

// The kernel's LDS bytes (the reference returns its shared-memory size, kkt:272).
extern "C" int reax_kkt_smem(void) { return (int)sizeof(reax::KktLds); }
