// Gated-DeltaNet chunk solve for gfx950: per 64-token chunk of a sequence and per value head,
//   A = (I + M)^-1,  M[r][c] = (k_r . k_c) * 2^(g[r] - g[c]) * beta[r] for c < r (both rows of the chunk), else 0,
// stored as bf16 rows of 64 (the lower block triangle of 16 x 16 blocks: columns up to the end of the row's own
// 16-column block; later columns are left untouched). Replaces reax_kkt, libreax_howu/reax_kkt.cu:263-272 (kernel
// kkt7_kernel, reax_kkt.cu:79-261): one key head's k k^T serves its two value heads (HV = 2H, kkt:265).
//
// The reference forms k k^T with bf16 tensor-core MMAs, the decay with the approximate ex2, the 16 x 16 diagonal
// inverses by forward substitution and the off-diagonal blocks with tf32 MMAs (10-bit mantissa operands). This build
// forms k k^T on the matrix cores too (bf16 products are exact, fp32 accumulation) and the rest in fp32 (v_exp_f32,
// the same blocked scheme with full fp32 products), so its results are at least as close to the exact inverse;
// agreement with the reference is to its own tf32/bf16 accuracy, not bit for bit.
//
// Layout: a persistent grid of three 256-thread workgroups per CU, each taking (chunk, key head) items in turn and
// loading the next item's k, g and beta into registers while it solves the current one. Per item: phase 1 stages k
// (64 x 128 bf16, 16-byte units XOR-swizzled by row), g and beta in LDS; phase 2 forms k k^T with
// v_mfma_f32_32x32x16_bf16 (wavefronts 0-2: the two diagonal 32 x 32 tiles and the one below them) and writes M for
// both value heads straight from the accumulators (decay, mask and beta) into fp32 16 x 16 blocks; phase 3 inverts
// the four diagonal blocks by forward substitution (a column per thread), then forms the blocks below them block
// row by block row with 4-column micro-tiles on all four wavefronts. 38 KB of LDS (k's staging area is reused for
// the inverse's blocks).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#pragma GCC visibility push(default)
#include "libreax_howu.h"
#pragma GCC visibility pop

#include "fmha_common.h"
#include "fmha_launch.h"

namespace reax {
namespace {

constexpr int KKT_BT = 64, KKT_K = 128, KKT_THREADS = 256;
// Workgroups per compute unit of the persistent grid: 3 leaves 170 VGPRs per lane for the solve plus the next item's
// prefetched k (at 4, 128 VGPRs, it spilled; measured 0.047 against 0.040 ms).
constexpr int KKT_WG_PER_CU = 3;

__device__ __forceinline__ uint16_t bf16_bits(float x) { return (uint16_t)(pack_bf16x2(x, 0.f) & 0xffffu); }

// fp32 16 x 16 blocks, row-major with the row's four 16-byte units XOR-swizzled by (row / 4) % 4: the micro-tile
// reads below (16 rows' unit q at once, or one row's 4 units) then touch 64 distinct banks.
__device__ __forceinline__ int bsw(int r, int c) { return r * 16 + ((((c >> 2) ^ (r >> 2)) & 3) << 2) + (c & 3); }
__device__ __forceinline__ f32x4_t bunit(const float* blk, int r, int q) {
  return *reinterpret_cast<const f32x4_t*>(blk + r * 16 + (((q ^ (r >> 2)) & 3) << 2));
}
// index of block (i, k), i > k, among the 6 blocks below the diagonal blocks: (1,0) (2,0) (2,1) (3,0) (3,1) (3,2)
__host__ __device__ constexpr int lidx(int i, int k) { return i * (i - 1) / 2 + k; }

struct KktLds {
  float mdiag[2][4][256];  // M's diagonal 16 x 16 blocks per value head; later the current round's T blocks
  float mlow[2][6][256];   // M's blocks below the diagonal blocks
  float mup[256];          // where the k k^T tiles' entries above the diagonal blocks go (never read)
  union {
    struct {
      uint16_t k[KKT_BT * KKT_K];  // k rows, 16-byte units XOR-swizzled by row
      float g[2][KKT_BT];
      float beta[2][KKT_BT];
    } in;  // phases 1-2
    struct {
      float d[2][4][256];  // D_b = (I + M_bb)^-1
      float a[2][3][256];  // A_10, A_20, A_21 (A_3j are only written out)
    } out;  // phase 3
  } u;
};

// element (r, c) of the staged k: 16 units of 8 per row, unit index XOR row % 16
__device__ __forceinline__ int ksw(int r, int c) { return r * KKT_K + ((((c >> 3) ^ (r & 15))) << 3) + (c & 7); }

// Persistent: workgroup b takes items b, b + gridDim.x, ... (item = kh * NT + chunk index) and loads the next item's
// k, g and beta into registers while it solves the current one.
__global__ void __launch_bounds__(KKT_THREADS, KKT_WG_PER_CU) kkt_kernel(const uint16_t* __restrict__ k, const float* __restrict__ g,
                                                             const uint16_t* __restrict__ beta, uint16_t* __restrict__ A,
                                                             const int64_t* __restrict__ cu,
                                                             const int64_t* __restrict__ cidx, int NT, int H, int HV) {
  __shared__ __align__(16) KktLds S;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int items = NT * H;
  struct Item {
    long long bos;
    int t0, nval, kh;
  };
  auto locate = [&](int it) {
    const int ch = it % NT, kh_ = it / NT;
    const int i_n = (int)cidx[2 * (long long)ch], i_t = (int)cidx[2 * (long long)ch + 1];
    const long long b0 = cu[i_n];
    const int t0_ = i_t * KKT_BT;
    return Item{b0, t0_, min(KKT_BT, (int)(cu[i_n + 1] - b0) - t0_), kh_};
  };
  // k rows (rows past the chunk's end read its last row; zeroed when staged), g and beta of the two value heads
  constexpr int KLD = KKT_BT * (KKT_K / 8) / KKT_THREADS;
  u32x4_t kp[KLD];
  float gp = 0.f;
  uint16_t bp = 0;
  auto fetch = [&](const Item& q) {
#pragma unroll
    for (int e = 0; e < KLD; ++e) {
      const int i = tid + KKT_THREADS * e, r = i >> 4, c8 = (i & 15) * 8;
      kp[e] = *reinterpret_cast<const u32x4_t*>(k + ((q.bos + q.t0 + min(r, q.nval - 1)) * H + q.kh) * KKT_K + c8);
    }
    if (tid < 2 * KKT_BT) {
      const long long row = (q.bos + q.t0 + min(tid & 63, q.nval - 1)) * HV + 2 * q.kh + (tid >> 6);
      gp = g[row];
      bp = beta[row];
    }
  };
  int item = (int)blockIdx.x;
  if (item < items) fetch(locate(item));
  for (; item < items; item += (int)gridDim.x) {
  // the thread index passes through an empty asm so that the compiler derives the per-lane LDS addresses inside
  // the loop instead of holding them all in registers across it
  int tid_ = threadIdx.x;
  asm volatile("" : "+v"(tid_));
  const int tid = tid_, lane = tid & 63;
  const Item cur = locate(item);
  const long long bos = cur.bos;
  const int t0 = cur.t0, nval = cur.nval, kh = cur.kh;
  const long long rs = (long long)HV * KKT_BT;  // A row stride (elements)
  uint16_t* const Abase = A + ((bos + t0) * HV + 2 * kh) * KKT_BT;  // row 0 of the chunk, value head 2 kh

  // ---- phase 1: the prefetched k rows (zero beyond the chunk's valid rows), g and beta into LDS
#pragma unroll
  for (int e = 0; e < KLD; ++e) {
    const int i = tid + KKT_THREADS * e, r = i >> 4, c8 = (i & 15) * 8;
    const u32x4_t zero4 = {0u, 0u, 0u, 0u};
    *reinterpret_cast<u32x4_t*>(S.u.in.k + ksw(r, c8)) = r < nval ? kp[e] : zero4;
  }
  if (tid < 2 * KKT_BT) {
    const int v = tid >> 6, r = tid & 63;
    S.u.in.g[v][r] = r < nval ? gp : 0.f;
    S.u.in.beta[v][r] = r < nval ? __uint_as_float((uint32_t)bp << 16) : 0.f;
  }
  __syncthreads();
  if (item + (int)gridDim.x < items) fetch(locate(item + (int)gridDim.x));

  // ---- phase 2: k k^T on the matrix cores for the tiles on and below the diagonal (wavefront 0: rows and columns
  // 0-31, 1: rows 32-63 x columns 0-31, 2: rows and columns 32-63), then M[v][r][c] = (k_r . k_c) 2^(g_r - g_c)
  // beta_r for c < r < nval, else 0, into the 16 x 16 blocks on and below the diagonal (the diagonal solve reads
  // only the strictly lower part of its block)
  if (wv < 3) {
    const int I = wv == 0 ? 0 : 1, J = wv == 2 ? 1 : 0;
    const int rr = lane & 31, kq = 8 * (lane >> 5);
    f32x16_t acc = {};
#pragma unroll
    for (int s = 0; s < KKT_K / 16; ++s) {
      const bf16x8_t a = as_bf16x8(*reinterpret_cast<const u32x4_t*>(S.u.in.k + ksw(32 * I + rr, 16 * s + kq)));
      const bf16x8_t b = as_bf16x8(*reinterpret_cast<const u32x4_t*>(S.u.in.k + ksw(32 * J + rr, 16 * s + kq)));
      acc = mfma32(a, b, acc);
    }
    // this lane's column c and rows r = 32 I + 8 jj + 4 (lane / 32) + 0..3 (jj = 0..3): g and beta as float4 runs
    const int c = 32 * J + rr, bc = c >> 4;
    const float gc[2] = {S.u.in.g[0][c], S.u.in.g[1][c]};
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int r0 = 32 * I + 8 * jj + 4 * (lane >> 5), br = r0 >> 4;
#pragma unroll
      for (int v = 0; v < 2; ++v) {
        const f32x4_t gr = *reinterpret_cast<const f32x4_t*>(&S.u.in.g[v][r0]);
        const f32x4_t b4 = *reinterpret_cast<const f32x4_t*>(&S.u.in.beta[v][r0]);
        float* blk = bc > br ? S.mup : br == bc ? S.mdiag[v][br] : S.mlow[v][lidx(br, bc)];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = r0 + e;
          const bool live = c < r && r < nval;
          blk[bsw(r & 15, c & 15)] = live ? (acc[4 * jj + e] * fast_exp2(gr[e] - gc[v])) * b4[e] : 0.f;
        }
      }
    }
  }
  __syncthreads();

  // ---- phase 3, blocked: (I + M)^-1 with 16 x 16 blocks. The diagonal blocks' inverses D_b by forward
  // substitution, one column j per thread (x_j = 1, x_r = 0 for r < j, x_r = -sum_{j<=c<r} M[r][c] x_c), then
  // block row by block row A_ij = -D_i T_ij, T_ij = sum_{k=j}^{i-1} M_ik A_kj (A_jj = D_j). Entry (r, c) of A goes
  // to A row r for r < nval and c up to the end of row r's own 16-column block; later columns are left untouched.
  if (tid < 128) {
    const int v = tid >> 6, bb = (tid >> 4) & 3, j = tid & 15;
    const float* M = S.mdiag[v][bb];
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int c = 0; c < r; ++c) {
        if (c & 1)
          s1 = __builtin_fmaf(M[bsw(r, c)], x[c], s1);
        else
          s0 = __builtin_fmaf(M[bsw(r, c)], x[c], s0);
      }
      x[r] = r < j ? 0.f : r == j ? 1.f : 0.f - (s0 + s1);  // 0 - s: an exact zero is stored as +0
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) S.u.out.d[v][bb][bsw(r, j)] = x[r];
  }
  __syncthreads();

  // Micro-tile of a 16 x 16 block per lane: row r = lane / 4, columns 4q .. 4q + 3 (q = lane % 4).
  const int mr = lane >> 2, mq = lane & 3;
  // bf16 of 4 adjacent entries of row (16 i + mr), columns 16 j + 4 mq.., of value head v, if the row is valid
  auto store4 = [&](int v, int i, int j, const f32x4_t y) {
    const int row = 16 * i + mr;
    if (row < nval) {
      uint32_t* dst = reinterpret_cast<uint32_t*>(Abase + row * rs + v * KKT_BT + 16 * j + 4 * mq);
      dst[0] = pack_bf16x2(y[0], y[1]);
      dst[1] = pack_bf16x2(y[2], y[3]);
    }
  };
  // acc += L[mr][.] X[.][4 mq ..] over the 16 inner indices
  auto mac = [&](f32x4_t& acc, const float* L, const float* X) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const f32x4_t l = bunit(L, mr, u);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f32x4_t xr = bunit(X, 4 * u + e, mq);
#pragma unroll
        for (int n = 0; n < 4; ++n) acc[n] = __builtin_fmaf(l[e], xr[n], acc[n]);
      }
    }
  };
  auto X = [&](int v, int kk, int j) -> const float* { return kk == j ? S.u.out.d[v][j] : S.u.out.a[v][lidx(kk, j)]; };

#pragma unroll
  for (int i = 1; i < 4; ++i) {
    // T_ij for the 2 i blocks (value head v, column block j) of this block row; wavefront w takes blocks w, w + 4
    // (in the order (v, j) = (0, 0), (1, 0), (0, 1), (1, 1), ...: the heavier j = 0 blocks pair with the lightest)
#pragma unroll
    for (int blk = wv; blk < 2 * i; blk += 4) {
      const int v = blk & 1, j = blk >> 1;
      f32x4_t t = {0.f, 0.f, 0.f, 0.f};
      for (int kk = j; kk < i; ++kk) mac(t, S.mlow[v][lidx(i, kk)], X(v, kk, j));
      *reinterpret_cast<f32x4_t*>(S.mdiag[v][j] + mr * 16 + (((mq ^ (mr >> 2)) & 3) << 2)) = t;
    }
    if (i == 1 && wv >= 2) {  // meanwhile the idle wavefronts write the diagonal blocks out
#pragma unroll
      for (int bb = 0; bb < 4; ++bb) store4(wv - 2, bb, bb, bunit(S.u.out.d[wv - 2][bb], mr, mq));
    }
    __syncthreads();
    // A_ij = -D_i T_ij
#pragma unroll
    for (int blk = wv; blk < 2 * i; blk += 4) {
      const int v = blk & 1, j = blk >> 1;
      f32x4_t y = {0.f, 0.f, 0.f, 0.f};
      mac(y, S.u.out.d[v][i], S.mdiag[v][j]);
#pragma unroll
      for (int n = 0; n < 4; ++n) y[n] = 0.f - y[n];
      if (i < 3) *reinterpret_cast<f32x4_t*>(S.u.out.a[v][lidx(i, j)] + mr * 16 + (((mq ^ (mr >> 2)) & 3) << 2)) = y;
      store4(v, i, j, y);
    }
    __syncthreads();  // (after the last block row: LDS is free for the next item)
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
  // persistent grid: KKT_WG_PER_CU workgroups per compute unit (the LDS and register budget), at most one per item
  const long long items = (long long)NT * H;
  if (items > INT32_MAX) return (int)hipErrorInvalidConfiguration;
  const int cus = device_cus(static_cast<hipStream_t>(stream));
  const int nwg = (int)(cus > 0 ? std::min<long long>(items, (long long)KKT_WG_PER_CU * cus) : items);
  hipLaunchKernelGGL(kkt_kernel, dim3((unsigned)nwg), dim3(KKT_THREADS), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(k), static_cast<const float*>(g), static_cast<const uint16_t*>(beta),
                     static_cast<uint16_t*>(A), static_cast<const int64_t*>(cu), static_cast<const int64_t*>(cidx), NT,
                     H, HV);
  return (int)hipGetLastError();
}

// The kernel's LDS bytes (the reference returns its shared-memory size, kkt:272).
extern "C" int reax_kkt_smem(void) { return (int)sizeof(reax::KktLds); }
