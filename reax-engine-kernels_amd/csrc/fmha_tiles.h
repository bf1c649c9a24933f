// Shared building blocks of the gfx950 attention kernels: K/V tile geometry, the LDS swizzle, direct-to-LDS tile
// loads, MFMA operand addressing and the wavefront reductions.
#pragma once
#include <climits>

#include "fmha_common.h"

namespace reax {

template <int HD>
struct FwdTile {
  static constexpr int BM = 128;       // folded query rows per workgroup (4 wavefronts x 32)
  static constexpr int BN = 64;        // keys per K/V tile
  static constexpr int NT = 256;       // threads per workgroup
  static constexpr int KU = HD / 8;    // 16-byte units per K/V row
  static constexpr int TILE = BN * HD * 2;  // bytes of one K or V tile
  static constexpr int DMA = TILE / 1024;   // 64-lane x 16-byte direct-to-LDS loads per tile
  static constexpr int DMA_W = DMA / 4;     // ... per wavefront
  static constexpr int QK = HD / 16;        // MFMA k-steps of S^T = K Q^T
  static constexpr int DB = HD / 32;        // 32-dim blocks of O^T
  static_assert(HD == 128 || HD == 256, "head_dim 128 or 256");
};

// Row-major K/V tiles with a 16-byte-unit XOR swizzle for gfx950's 64-bank LDS (256 bytes per access phase):
//   - K operand reads (ds_read_b128, 16 lanes per phase) touch 16 consecutive rows at one unit: f() is a
//     bijection on r mod 16, so the 16 units land in 16 distinct bank groups;
//   - transposed V reads (ds_read_b64_tr_b16, 32 lanes per phase) touch 4 consecutive rows x 4 adjacent units:
//     bits 2-3 of f() (= r & 3) differ across the 4 rows, so the 16 (row, unit) pieces are distinct.
// Unit u of row r sits at byte r * (HD * 2) + ((u ^ swz(r)) << 4) of the tile.
__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

__device__ __forceinline__ u32x4_t ld16(const uint16_t* p) { return *reinterpret_cast<const u32x4_t*>(p); }

#define REAX_LDS(p) ((__attribute__((address_space(3))) void*)(p))

// One 16-byte direct global -> LDS load per lane (global_load_lds_dwordx4): lane l's bytes land at lds + 16 l.
__device__ __forceinline__ void lds_dma16(const void* src, uint8_t* lds) {
  __builtin_amdgcn_global_load_lds(src, REAX_LDS(lds), 16, 0, 0);
}

// The same load issued as inline assembly. The compiler keeps no direct-to-LDS bookkeeping for inline assembly:
// with the builtin it tracks the load, and its wait insertion then drains the LDS counter completely
// (lgkmcnt(0)) before MFMAs whose operands come from LDS, instead of waiting only for the reads each one needs;
// with the assembly form it also adds no conservative vmcnt(0) before LDS reads of other buffers. The caller
// orders the load explicitly: s_waitcnt vmcnt before reading the destination, lgkmcnt(0) after the last read of a
// region before loading into it again. NT adds the nontemporal hint, for data read exactly once (the K/V stream
// of a decode step): measured on MI355X, a cold streaming read with nt runs at ~6.8 TB/s against ~3.9 TB/s
// without it when the caches hold dirty lines.
template <bool NT>
__device__ __forceinline__ void lds_dma16_asm(const void* src, uint8_t* lds) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)reinterpret_cast<uintptr_t>(lds));
  if (NT)
    asm volatile("global_load_lds_dwordx4 %0, off nt" ::"v"(src), "{m0}"(m0) : "memory");
  else
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(m0) : "memory");
}

// Direct global -> LDS copy of a K or V tile. Load c of a tile fills bytes [c*1024, c*1024 + 1024): lane l
// lands at c*1024 + 16 l, i.e. row r, swizzled unit pu, and fetches the logical unit u = pu ^ swz(r) of that
// row. With NWV wavefronts per workgroup, wavefront w issues loads c = w*DW .. w*DW + DW - 1 (DW = loads per
// tile / NWV). BN is the tile's key count.
template <int HD, int NWV, int BN = FwdTile<HD>::BN>
struct Dma {
  static constexpr int LOADS = BN * HD * 2 / 1024;
  static constexpr int DW = LOADS / NWV;
  static_assert(DW >= 1 && DW * NWV == LOADS, "tile loads split evenly over the wavefronts");
  uint32_t off[DW];  // byte offset of this lane's source relative to the tile's first key row

  __device__ __forceinline__ static void slot(int w, int i, int lane, int& r, int& u) {
    const int byte = (w * DW + i) * 1024 + 16 * lane;
    r = byte / (HD * 2);
    u = ((byte % (HD * 2)) >> 4) ^ swz(r);
  }
  __device__ __forceinline__ Dma(long long stride, int w, int lane) {
#pragma unroll
    for (int i = 0; i < DW; ++i) {
      int r, u;
      slot(w, i, lane, r, u);
      off[i] = (uint32_t)((long long)r * stride * 2 + 16 * u);
    }
  }
  // One of the DW loads of tile(): load i only, so that a caller can spread a tile's loads over time.
  template <int KIND = 0>
  __device__ __forceinline__ void load_one(int i, uint8_t* buf, const uint16_t* base, long long stride, bool fast,
                                           int k0, int kend, int w, int lane) const {
    // The per-lane inputs pass through empty asm so that the compiler derives the addresses here, where the
    // load is issued, instead of keeping them live (or spilled) from the kernel's start.
    const uint8_t* src;
    if (fast && k0 + BN <= kend) {
      uint32_t o = off[i];
      asm volatile("" : "+v"(o));
      src = reinterpret_cast<const uint8_t*>(base + (long long)k0 * stride) + o;
    } else {
      int r, u, ln = lane;
      asm volatile("" : "+v"(ln));
      slot(w, i, ln, r, u);
      const int key = min(k0 + r, kend - 1);
      src = reinterpret_cast<const uint8_t*>(base + (long long)key * stride + 8 * u);
    }
    if (KIND)
      lds_dma16_asm<KIND == 2>(src, buf + (w * DW + i) * 1024);
    else
      lds_dma16(src, buf + (w * DW + i) * 1024);
  }
  // Copies the tile at key k0. Full tiles (k0 + BN <= kend, and 32-bit row offsets) use the precomputed
  // offsets; a partial last tile clamps its rows to the window's last key: those scores are masked, so they
  // only ever meet a zero probability.
  // KIND 0: builtin load; 1: inline-assembly load; 2: inline-assembly nontemporal load
  template <int KIND = 0>
  __device__ __forceinline__ void tile(uint8_t* buf, const uint16_t* base, long long stride, bool fast, int k0,
                                       int kend, int w, int lane) const {
    if (fast && k0 + BN <= kend) {
      const uint16_t* tb = base + (long long)k0 * stride;
#pragma unroll
      for (int i = 0; i < DW; ++i) {
        const uint8_t* src = reinterpret_cast<const uint8_t*>(tb) + off[i];
        if (KIND)
          lds_dma16_asm<KIND == 2>(src, buf + (w * DW + i) * 1024);
        else
          lds_dma16(src, buf + (w * DW + i) * 1024);
      }
    } else {
#pragma unroll
      for (int i = 0; i < DW; ++i) {
        int r, u;
        slot(w, i, lane, r, u);
        const int key = min(k0 + r, kend - 1);
        if (KIND)
          lds_dma16_asm<KIND == 2>(base + (long long)key * stride + 8 * u, buf + (w * DW + i) * 1024);
        else
          lds_dma16(base + (long long)key * stride + 8 * u, buf + (w * DW + i) * 1024);
      }
    }
  }
};

// f(std::integral_constant<int, I>) for I = B .. E-1, expanded at compile time (a 32-step "#pragma unroll" loop
// over a long interleaved block exceeds the unroller's size limit and would stay a loop with dynamic indexing)
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// Workgroup barrier that orders execution only. __syncthreads() also fences memory, which makes every wavefront
// wait at the barrier for its in-flight direct-to-LDS loads (vmcnt(0)); the memory clobber keeps the compiler
// from moving memory accesses across this one.
__device__ __forceinline__ void exec_barrier() { asm volatile("s_barrier" ::: "memory"); }

__device__ __forceinline__ void wait_dma_and_sync() {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wavefront's direct-to-LDS loads have landed
  __syncthreads();                     // ... and every other wavefront's
}

// LDS read addresses. Row offsets (multiples of HD*2) and the swizzled 16-byte unit (bits 4..8) occupy disjoint
// bits, so every operand address is a per-lane base XOR a compile-time constant (plus a constant offset).
//   K operand (kb, ks): row 32kb + lr, unit 2ks + hf  ->  kbase[kb] ^ (32 ks)
//   V operand (db, ss, second half): row 16ss + 4h + i/4 + 8*second, unit 4db + 2dh + (i&3)/2, byte 8(i&1)
//     -> (16ss + 8 second)*HD*2 + (vbase ^ vconst(db, second))
template <int HD>
__device__ __forceinline__ uint32_t k_lane_base(int kb, int lr, int hf) {
  const int r = 32 * kb + lr;
  return (uint32_t)(r * HD * 2 + ((hf ^ swz(r)) << 4));
}
// With row = 16ss + 4h + i/4 + 8 second, swz(row) = ((i/4) << 2) | h | (second << 1) and the unit is
// 4db + 2dh + (i&3)/2, so unit ^ swz(row) = L(lane) ^ C(db, second) with the two parts below.
template <int HD>
__device__ __forceinline__ uint32_t v_lane_base(int lane) {
  const int h = lane >> 5, dh = (lane >> 4) & 1, i = lane & 15;
  const int L = (((i >> 1) & 1) ^ h) | (dh << 1) | (((i >> 2) & 3) << 2);
  return (uint32_t)((4 * h + (i >> 2)) * HD * 2 + (L << 4) + 8 * (i & 1));
}
__device__ __forceinline__ constexpr uint32_t v_const(int db, int second) {
  return (uint32_t)(((second << 1) | ((db & 3) << 2) | (((db >> 2) & 1) << 4)) << 4);
}

// S^T for one 64-key tile: s[kb][v] = score of this lane's row against key 32kb + 8(v/4) + 4hf + v%4.
template <int HD>
__device__ __forceinline__ void qk_tile(f32x16_t (&s)[2], const uint8_t* kbuf, const bf16x8_t (&qf)[HD / 16],
                                        const uint32_t (&kbase)[2]) {
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int e = 0; e < 16; ++e) s[kb][e] = 0.f;
#pragma unroll
    for (int ks = 0; ks < HD / 16; ++ks) {
      const u32x4_t kf = *reinterpret_cast<const u32x4_t*>(kbuf + (kbase[kb] ^ (32u * ks)));
      s[kb] = mfma32(as_bf16x8(kf), qf[ks], s[kb]);
    }
  }
}

typedef short i16x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x2_t ds_read_tr16(const uint8_t* p) {
  const i16x4_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4_t*)(p));
  return __builtin_bit_cast(u32x2_t, a);
}

// V^T operand (32 dims x 16 keys in MFMA key order) of dim block db, k-step ss, from the row-major V tile with
// two ds_read_b64_tr_b16: in each 16-lane group, lane i reads 4 dims of key row i/4 and receives 4 keys of
// dim i back.
template <int HD>
__device__ __forceinline__ bf16x8_t v_operand(const uint8_t* vbuf, int db, int ss, uint32_t vbase) {
  const u32x2_t a = ds_read_tr16(vbuf + 16 * ss * HD * 2 + (vbase ^ v_const(db, 0)));
  const u32x2_t b = ds_read_tr16(vbuf + (16 * ss + 8) * HD * 2 + (vbase ^ v_const(db, 1)));
  return as_bf16x8(u32x4_t{a[0], a[1], b[0], b[1]});
}

__device__ __forceinline__ int wave_max(int x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x = max(x, __shfl_xor(x, off, 64));
  return x;
}
__device__ __forceinline__ int wave_min(int x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x = min(x, __shfl_xor(x, off, 64));
  return x;
}

// The same as a scalar, with DPP steps instead of six ds_bpermute round trips (all 64 lanes must be active):
// quad permutes [1,0,3,2] and [2,3,0,1] give each quad its extremum, row shifts by 4 and 8 carry it to lane 15 of
// each 16-lane row, and the row broadcasts of lane 15 (into rows 1 and 3) and lane 31 (into rows 2 and 3) leave
// the wavefront's extremum in lane 63, read back as a scalar. Lanes whose DPP source lies outside the row, or
// whose row is masked off, take the identity. (Used where a kernel's prologue waits on it; inside the larger
// kernels the DPP form raised register pressure into scratch spills.)
template <bool MAX>
__device__ __forceinline__ int wave_ext_dpp(int x) {
  constexpr int ID = MAX ? INT_MIN : INT_MAX;
  auto op = [](int a, int b) { return MAX ? max(a, b) : min(a, b); };
  x = op(x, __builtin_amdgcn_update_dpp(ID, x, 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
  x = op(x, __builtin_amdgcn_update_dpp(ID, x, 0x4E, 0xF, 0xF, false));   // quad_perm [2,3,0,1]
  x = op(x, __builtin_amdgcn_update_dpp(ID, x, 0x114, 0xF, 0xF, false));  // row_shr:4
  x = op(x, __builtin_amdgcn_update_dpp(ID, x, 0x118, 0xF, 0xF, false));  // row_shr:8
  x = op(x, __builtin_amdgcn_update_dpp(ID, x, 0x142, 0xA, 0xF, false));  // row_bcast:15
  x = op(x, __builtin_amdgcn_update_dpp(ID, x, 0x143, 0xC, 0xF, false));  // row_bcast:31
  return __builtin_amdgcn_readlane(x, 63);
}

// Lazy rescaling: the running max (log2 units) is raised only when a tile's max exceeds it by more than
// RESCALE_SLACK, so probabilities stay below 2^RESCALE_SLACK and the O / row-sum rescale is rare.
constexpr float RESCALE_SLACK = 8.0f;

}  // namespace reax
