// Gated-DeltaNet chunk solve for gfx950: per 64-token chunk of a sequence and per value head,
//   A = (I + M)^-1,  M[r][c] = (k_r . k_c) * 2^(g[r] - g[c]) * beta[r] for c < r (both rows of the chunk), else 0,
// stored as bf16 rows of 64 (the lower block triangle of 16 x 16 blocks: columns up to the end of the row's own
// 16-column block; later columns are left untouched). Replaces reax_kkt, libreax_howu/reax_kkt.cu:263-272 (kernel
// kkt7_kernel, reax_kkt.cu:79-261): one key head's k k^T serves its two value heads (HV = 2H, kkt:265).
//
// The reference forms k k^T with bf16 tensor-core MMAs, the decay with the approximate ex2, the 16 x 16 diagonal
// inverses by forward substitution and the off-diagonal blocks with tf32 MMAs (10-bit mantissa operands). This build
// computes the same quantities in fp32 throughout (exact bf16 products, v_exp_f32, full-precision forward
// substitution), so its results are at least as close to the exact inverse; agreement with the reference is to
// its own tf32/bf16 accuracy, not bit for bit.
//
// Layout: one workgroup of 256 threads per (chunk, key head). Phase 1 stages the chunk's k (64 x 128) in LDS as
// fp32; phase 2 forms the lower half of k k^T (each thread a 4 x 4 block, 128-long dot products); phase 3 applies
// decay, mask and beta for both value heads; phase 4 solves (I + M) X = I column by column (128 threads: 2 heads x
// 64 columns, the column in registers, M read by broadcast); phase 5 writes the bf16 rows.
#include <hip/hip_runtime.h>
#include <stdint.h>

#pragma GCC visibility push(default)
#include "libreax_howu.h"
#pragma GCC visibility pop

#include "fmha_common.h"

namespace reax {
namespace {

constexpr int KKT_BT = 64, KKT_K = 128, KKT_THREADS = 256;
constexpr int KKT_LD = KKT_BT + 1;  // padded row of the 64 x 64 fp32 matrices
constexpr int KKT_LDM = KKT_BT + 4;  // rows of M: 16-byte aligned, read 4 entries at a time by broadcast

struct KktLds {
  float k[KKT_BT][KKT_K + 4];  // padded rows: the 4 x 4 block reads of phase 2 spread over the banks
  float raw[KKT_BT][KKT_LD];
  float m[2][KKT_BT][KKT_LDM];
  float x[2][KKT_BT][KKT_LD];
  float g[2][KKT_BT];
  float beta[2][KKT_BT];
};

__global__ void __launch_bounds__(KKT_THREADS) kkt_kernel(const uint16_t* __restrict__ k, const float* __restrict__ g,
                                                          const uint16_t* __restrict__ beta, uint16_t* __restrict__ A,
                                                          const int64_t* __restrict__ cu,
                                                          const int64_t* __restrict__ cidx, int H, int HV) {
  __shared__ __align__(16) KktLds S;
  const int tid = threadIdx.x;
  const int i_n = (int)cidx[2 * (long long)blockIdx.x], i_t = (int)cidx[2 * (long long)blockIdx.x + 1];
  const int kh = blockIdx.y;
  const long long bos = cu[i_n];
  const int T = (int)(cu[i_n + 1] - bos);
  const int t0 = i_t * KKT_BT;
  const int nval = min(KKT_BT, T - t0);

  // ---- phase 1: k rows (zero beyond the chunk's valid rows), g and beta of the two value heads
  for (int i = tid; i < KKT_BT * (KKT_K / 8); i += KKT_THREADS) {
    const int r = i >> 4, c8 = (i & 15) * 8;
    u32x4_t w = {0u, 0u, 0u, 0u};
    if (r < nval) w = *reinterpret_cast<const u32x4_t*>(k + ((bos + t0 + r) * H + kh) * KKT_K + c8);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      S.k[r][c8 + 2 * q] = bf16lo(w[q]);
      S.k[r][c8 + 2 * q + 1] = bf16hi(w[q]);
    }
  }
  if (tid < 2 * KKT_BT) {
    const int v = tid >> 6, r = tid & 63, hv = 2 * kh + v;
    S.g[v][r] = r < nval ? g[(bos + t0 + r) * HV + hv] : 0.f;
    S.beta[v][r] = r < nval ? bf16lo(beta[(bos + t0 + r) * HV + hv]) : 0.f;
  }
  __syncthreads();

  // ---- phase 2: raw = k k^T on and below the diagonal, a 4 x 4 block per thread
  {
    const int bi = tid >> 4, bj = tid & 15;
    if (bj <= bi) {
      float acc[4][4];
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = 0.f;
      for (int c = 0; c < KKT_K; c += 4) {
        f32x4_t ra[4], rb[4];
#pragma unroll
        for (int a = 0; a < 4; ++a) ra[a] = *reinterpret_cast<const f32x4_t*>(&S.k[4 * bi + a][c]);
#pragma unroll
        for (int b = 0; b < 4; ++b) rb[b] = *reinterpret_cast<const f32x4_t*>(&S.k[4 * bj + b][c]);
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int b = 0; b < 4; ++b) acc[a][b] = __builtin_fmaf(ra[a][e], rb[b][e], acc[a][b]);
      }
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) S.raw[4 * bi + a][4 * bj + b] = acc[a][b];
    }
  }
  __syncthreads();

  // ---- phase 3: M for both value heads (strictly lower, valid rows only): raw * 2^(g_r - g_c) * beta_r
  for (int i = tid; i < 2 * KKT_BT * KKT_BT; i += KKT_THREADS) {
    const int v = i >> 12, r = (i >> 6) & 63, c = i & 63;
    float m = 0.f;
    if (c < r && r < nval) m = (S.raw[r][c] * fast_exp2(S.g[v][r] - S.g[v][c])) * S.beta[v][r];
    S.m[v][r][c] = m;
  }
  __syncthreads();

  // ---- phase 4: (I + M) X = I by forward substitution, one column j per thread: x_j = 1, x_r = 0 for r < j,
  // x_r = -sum_{c<r} M[r][c] x_c for r > j (the terms with c < j vanish)
  if (tid < 2 * KKT_BT) {
    const int v = tid >> 6, j = tid & 63;
    const float(*M)[KKT_LDM] = S.m[v];
    float x[KKT_BT];
#pragma unroll
    for (int r = 0; r < KKT_BT; ++r) {
      float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
      for (int c = 0; c + 3 < r; c += 4) {
        const f32x4_t mr = *reinterpret_cast<const f32x4_t*>(&M[r][c]);
        s0 = __builtin_fmaf(mr[0], x[c], s0);
        s1 = __builtin_fmaf(mr[1], x[c + 1], s1);
        s2 = __builtin_fmaf(mr[2], x[c + 2], s2);
        s3 = __builtin_fmaf(mr[3], x[c + 3], s3);
      }
#pragma unroll
      for (int c = r & ~3; c < r; ++c) s0 = __builtin_fmaf(M[r][c], x[c], s0);
      const float s = (s0 + s1) + (s2 + s3);
      x[r] = r < j ? 0.f : r == j ? 1.f : 0.f - s;  // 0 - s: an exact zero is stored as +0
    }
#pragma unroll
    for (int r = 0; r < KKT_BT; ++r) S.x[v][r][j] = x[r];
  }
  __syncthreads();

  // ---- phase 5: rows r < nval, columns up to the end of the row's 16-column block, as bf16 pairs
  for (int i = tid; i < 2 * KKT_BT * (KKT_BT / 2); i += KKT_THREADS) {
    const int v = i >> 11, r = (i >> 5) & 63, c2 = (i & 31) * 2;
    if (r >= nval || c2 >= 16 * (r / 16 + 1)) continue;
    const int hv = 2 * kh + v;
    *reinterpret_cast<uint32_t*>(A + ((bos + t0 + r) * HV + hv) * KKT_BT + c2) =
        pack_bf16x2(S.x[v][r][c2], S.x[v][r][c2 + 1]);
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
