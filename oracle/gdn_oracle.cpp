// CPU oracle for the norm kernels of libreax_howu.so outside the attention path.
//
// TEST INFRASTRUCTURE ONLY. This file is the checker, never the product: only tests/ (and the smoke check in
// __graft_entry__.py) may load the library built from it. It is compiled with -ffp-contract=off so that every
// fp32 operation below rounds exactly as written (the reference is built with nvcc -fmad=false, build.sh:17-18).
//
// rarn_ref restates libreax_howu/reax_rarn_final.cu (reduce-add RMSNorm, D = 2560), element by element, in the
// reference's rounding order:
//   d = part[0]; d = d + part[s] for s = 1..S-1 (serial: bf16 round after every add); d = bf16(d)  (rarn:47-54)
//   h = bf16(res + d)                                                                               (rarn:55)
//   a[c] = sum over chunks k = 0..19 in order of h[128k + c]^2, c = 0..127 (product rounded)        (rarn:57-58)
//   slot m = ((a[4m] + a[4m+1]) + a[4m+2]) + a[4m+3], m = 0..31                                      (rarn:63-66)
//   tree: t(m) = s(m) + s(m+16) (m < 16), then + 8, + 4, + 2, + 1                                    (rarn:67-78)
//   r = 1 / sqrt(tot * factor + eps)                                                                 (rarn:82)
//   out = bf16((h * r) * (1 + w))                                                                    (rarn:86-87)
// The reference evaluates r with CUDA's approximate rsqrtf; this oracle (like the HIP kernel) evaluates it in
// double precision and rounds to fp32: bit-exact agreement with the reference at that step is not claimed.
#include <cmath>
#include <cstdint>
#include <cstring>

namespace {

inline float bf2f(uint16_t b) {
  const uint32_t u = (uint32_t)b << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
// fp32 -> bf16 round-to-nearest-even (NaN kept quiet)
inline uint16_t f2bf(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
inline float bfr(float x) { return bf2f(f2bf(x)); }

constexpr int D = 2560, CH = 20;

}  // namespace

extern "C" {

// Returns the reference's codes: 0 for n <= 0, -1 for D != 2560, -2 for S outside 2..8, else 0 after computing.
// mutant != 0 plants a deliberate mistake (used only to show that the pinning tests catch it):
//   1: sum of squares accumulated in a plain row-major sequential order instead of the reference's tree
//   2: (1 + w) replaced by w
//   3: d not rounded to bf16 before adding the residual
// r_out (may be null) receives each row's r.
int oracle_rarn(const uint16_t* part, int S, int serial, long long pstride, const uint16_t* res, const uint16_t* w,
                uint16_t* h_out, uint16_t* out, int n, int d, float eps, float factor, int mutant, float* r_out) {
  if (d != D || n <= 0) return n <= 0 ? 0 : -1;
  if (S < 2 || S > 8) return -2;
  for (long long row = 0; row < n; ++row) {
    const long long ro = row * D;
    float hrow[D];
    for (int c = 0; c < D; ++c) {
      float x = bf2f(part[ro + c]);
      for (int s = 1; s < S; ++s) {
        x = x + bf2f(part[s * pstride + ro + c]);
        if (serial) x = bfr(x);
      }
      if (mutant != 3) x = bfr(x);
      const float h = bfr(bf2f(res[ro + c]) + x);
      hrow[c] = h;
      h_out[ro + c] = f2bf(h);
    }
    float tot;
    if (mutant == 1) {
      tot = 0.f;
      for (int c = 0; c < D; ++c) tot = tot + hrow[c] * hrow[c];
    } else {
      float a[128];
      for (int c = 0; c < 128; ++c) {
        a[c] = 0.f;
        for (int k = 0; k < CH; ++k) a[c] = a[c] + hrow[128 * k + c] * hrow[128 * k + c];
      }
      float sl[32];
      for (int m = 0; m < 32; ++m) sl[m] = ((a[4 * m] + a[4 * m + 1]) + a[4 * m + 2]) + a[4 * m + 3];
      for (int half = 16; half >= 1; half >>= 1)
        for (int m = 0; m < half; ++m) sl[m] = sl[m] + sl[m + half];
      tot = sl[0];
    }
    const float x = tot * factor + eps;
    const float r = (float)(1.0 / std::sqrt((double)x));
    if (r_out) r_out[row] = r;
    for (int c = 0; c < D; ++c) {
      const float wv = bf2f(w[c]);
      const float g = mutant == 2 ? wv : 1.f + wv;
      out[ro + c] = f2bf((hrow[c] * r) * g);
    }
  }
  return 0;
}

}  // extern "C"
