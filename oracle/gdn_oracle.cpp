// CPU oracle for the norm and conv kernels of libreax_howu.so outside the attention path.
//
// TEST INFRASTRUCTURE ONLY. This file is the checker, never the product: only tests/ (and the smoke check in
// __graft_entry__.py) may load the library built from it. It is compiled with -ffp-contract=off so that every
// fp32 operation below rounds exactly as written (the reference is built with nvcc -fmad=false, build.sh:17-18).
//
// oracle_rarn restates libreax_howu/reax_rarn_final.cu ("rarn" below; reduce-add RMSNorm, D = 2560), element by
// element, in the reference's rounding order:
//   d = part[0]; d = d + part[s] for s = 1..S-1 (serial: bf16 round after every add); d = bf16(d)  (rarn:47-54)
//   h = bf16(res + d)                                                                               (rarn:55)
//   a[c] = sum over chunks k = 0..19 in order of h[128k + c]^2, c = 0..127 (product rounded)        (rarn:57-58)
//   slot m = ((a[4m] + a[4m+1]) + a[4m+2]) + a[4m+3], m = 0..31                                      (rarn:63-66)
//   tree: t(m) = s(m) + s(m+16) (m < 16), then + 8, + 4, + 2, + 1                                    (rarn:67-78)
//   r = 1 / sqrt(tot * factor + eps)                                                                 (rarn:82)
//   out = bf16((h * r) * (1 + w))                                                                    (rarn:86-87)
// The reference evaluates r with CUDA's approximate rsqrtf; this oracle (like the HIP kernel) evaluates it in
// double precision and rounds to fp32: bit-exact agreement with the reference at that step is not claimed.
//
// oracle_kkt restates libreax_howu/reax_kkt.cu ("kkt" below; the Gated-DeltaNet chunk solve), in double precision:
//   per chunk (sequence i_n, chunk i_t of 64 tokens; cidx pairs) and key head kh, for value heads hv = 2kh, 2kh+1:
//   M[r][c] = (k_r . k_c) * 2^(g[r] - g[c]) * beta[r] for c < r < nval, else 0; g[r] - g[c] rounded to fp32 as the
//   reference subtracts in fp32 before ex2 (kkt:134-140); A = (I + M)^-1 (the diagonal-block inverses by forward
//   substitution and the block recurrence of kkt:170-240 compute exactly this lower-triangular inverse); rows r <
//   nval, columns up to the end of the row's 16-column block, stored as bf16 (kkt:191-199, 243-258).
// The reference's bf16 / tf32 tensor-core products and approximate ex2 make it agree with this to its own accuracy.
//
// oracle_howu restates libreax_howu/reax_howu.cu ("howu" below; the Gated-DeltaNet chunked forward, skip-A form):
//   per sequence and value head hv (key head hv / (HV/H)), state h [128 k][128 v] = 0; per 64-token chunk (g is the
//   chunk-local cumulative log2 decay, eg = 2^g):
//   vb = bf16(v beta); kb = bf16(bf16(k beta) eg)                                                  (howu:95-104, 146-156)
//   u = A vb, w = A kb over the lower block triangle of A; ub = bf16(u), wb = bf16(w)              (howu:131-163, 202-208)
//   AQ[t][s] = bf16((q_t . k_s) 2^(g_t - g_s)) for s <= t, both valid, else 0                        (howu:165-196)
//   vw = wb bf16(h), oi = q bf16(h); x = ub - vw; vn = bf16(x); vdec = bf16(x 2^(g_last - g_t))      (howu:210-244)
//   o = bf16(fma(AQ vn, scale, (oi 2^(g_t)) scale))                                                 (howu:256-283)
//   h = h 2^(g_last) + k^T vdec                                                                     (howu:285-300)
// Products are summed in double (the reference's tensor-core sums are fp32 in a hardware order). exact != 0 drops
// every bf16 rounding and uses the exact (I + M)^-1 computed here instead of the given A: that form must equal the
// token-by-token gated delta rule, which the tests check.
//
// oracle_conv restates libreax_howu/reax_conv_v2.cu ("conv" below; causal 4-tap conv1d + SiLU + L2 norm):
//   tap j = 0..3: src = meta.x - 3 + j, skipped when src < 0; row meta.z + src of qkv when src >= meta.y, else row
//   meta.w + src of the cache                                                                        (conv:88-92)
//   acc = fma(w[c][j], x, acc) over the taps in order, from 0                                        (conv:96-108)
//   y = bf16(acc); s = bf16(y / fp32(1 + exp(-y)))                                                   (conv:112-122)
//   q/k units: per 8-channel group p = s1*s1, then fma(s0, s0, p), fma(s2, s2, p) .. fma(s7, s7, p); the 16 groups
//   of a 128-channel unit combine by a butterfly over group distance 8, 4, 2, 1; rstd = 1 / sqrt(eps + sum);
//   out = bf16(rstd * s), written once (rep 1) or twice side by side (rep 2)                         (conv:123-142)
//   v units: out = s                                                                                 (conv:143-147)
// The reference evaluates exp, sqrt and the reciprocal with fast approximations (its exp restates libdevice's
// expf, which this project does not reproduce); the oracle, like the HIP kernel, evaluates 1 + exp(-y) and
// 1/sqrt in double precision and rounds them to fp32, so bit-exact agreement with the reference is not claimed
// for those steps.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

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

// mutant != 0 plants a deliberate mistake (used only to show that the pinning tests catch it):
//   1: the inter-chunk output term without its 2^(g_t) decay; 2: the intra-chunk causal mask strict (s < t);
//   3: the state carried without its chunk decay 2^(g_last); 4: vdec without the 2^(g_last - g_t) factor
int oracle_howu(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* beta, const uint16_t* A,
                const float* g, uint16_t* o, const int64_t* cu, float scale, int N, int H, int HV, int exact,
                int mutant) {
  if (H <= 0 || HV % H) return -1;
  const int rep = HV / H;
  auto rb = [&](double x) -> double { return exact ? x : (double)bf2f(f2bf((float)x)); };
  std::vector<double> h(128 * 128), Hs(128 * 128);
  std::vector<double> Ac(64 * 64), vb(64 * 128), kb(64 * 128), ub(64 * 128), wb(64 * 128), AQ(64 * 64);
  std::vector<double> vn(64 * 128), vdec(64 * 128), qf(64 * 128), kf(64 * 128);
  for (int i_n = 0; i_n < N; ++i_n) {
    const int64_t bos = cu[i_n];
    const int T = (int)(cu[i_n + 1] - bos);
    for (int hv = 0; hv < HV; ++hv) {
      const int kh = hv / rep;
      std::fill(h.begin(), h.end(), 0.0);
      for (int t0 = 0; t0 < T; t0 += 64) {
        const int nv = T - t0 < 64 ? T - t0 : 64;
        double G[64], eg[64], Bt[64];
        for (int t = 0; t < 64; ++t) {
          G[t] = t < nv ? (double)g[(bos + t0 + t) * HV + hv] : 0.0;
          eg[t] = std::exp2(G[t]);
          Bt[t] = t < nv ? (double)bf2f(beta[(bos + t0 + t) * HV + hv]) : 0.0;
        }
        for (int t = 0; t < 64; ++t)
          for (int d = 0; d < 128; ++d) {
            qf[t * 128 + d] = t < nv ? (double)bf2f(q[((bos + t0 + t) * H + kh) * 128 + d]) : 0.0;
            kf[t * 128 + d] = t < nv ? (double)bf2f(k[((bos + t0 + t) * H + kh) * 128 + d]) : 0.0;
            const double vv = t < nv ? (double)bf2f(v[((bos + t0 + t) * HV + hv) * 128 + d]) : 0.0;
            vb[t * 128 + d] = rb(vv * Bt[t]);
            kb[t * 128 + d] = rb(rb(kf[t * 128 + d] * Bt[t]) * eg[t]);
          }
        // A: the given bf16 lower block triangle (upper blocks read as 0), or the exact inverse
        if (exact) {
          double M[64][64];
          for (int r = 0; r < 64; ++r)
            for (int c = 0; c < 64; ++c) {
              M[r][c] = 0.0;
              if (c < r && r < nv) {
                double dot = 0.0;
                for (int d = 0; d < 128; ++d) dot += kf[r * 128 + d] * kf[c * 128 + d];
                M[r][c] = dot * std::exp2(G[r] - G[c]) * Bt[r];
              }
            }
          for (int j = 0; j < 64; ++j)
            for (int r = 0; r < 64; ++r) {
              if (r < j) { Ac[r * 64 + j] = 0.0; continue; }
              double sacc = 0.0;
              for (int c = j; c < r; ++c) sacc += M[r][c] * Ac[c * 64 + j];
              Ac[r * 64 + j] = r == j ? 1.0 : -sacc;
            }
        } else {
          for (int r = 0; r < 64; ++r)
            for (int c = 0; c < 64; ++c)
              Ac[r * 64 + c] = (r < nv && c / 16 <= r / 16) ? (double)bf2f(A[((bos + t0 + r) * HV + hv) * 64 + c]) : 0.0;
        }
        for (int t = 0; t < 64; ++t)
          for (int c = 0; c < 128; ++c) {
            double su = 0.0, sw = 0.0;
            for (int s2 = 0; s2 < 64; ++s2) {
              su += Ac[t * 64 + s2] * vb[s2 * 128 + c];
              sw += Ac[t * 64 + s2] * kb[s2 * 128 + c];
            }
            ub[t * 128 + c] = rb(su);
            wb[t * 128 + c] = rb(sw);
          }
        for (int t = 0; t < 64; ++t)
          for (int s2 = 0; s2 < 64; ++s2) {
            double z = 0.0;
            const bool in = mutant == 2 ? s2 < t : s2 <= t;
            if (in && t < nv && s2 < nv) {
              double dot = 0.0;
              for (int d = 0; d < 128; ++d) dot += qf[t * 128 + d] * kf[s2 * 128 + d];
              z = rb(dot * std::exp2((double)((float)G[t] - (float)G[s2])));
            }
            AQ[t * 64 + s2] = z;
          }
        for (int i = 0; i < 128 * 128; ++i) Hs[i] = rb(h[i]);
        const double glast = G[nv - 1];
        for (int t = 0; t < 64; ++t) {
          const double da = t < nv ? (mutant == 4 ? 1.0 : std::exp2(glast - G[t])) : 0.0;
          for (int c = 0; c < 128; ++c) {
            double vw = 0.0;
            for (int d = 0; d < 128; ++d) vw += wb[t * 128 + d] * Hs[d * 128 + c];
            const double x = ub[t * 128 + c] - vw;
            vn[t * 128 + c] = rb(x);
            vdec[t * 128 + c] = rb(x * da);
          }
        }
        for (int t = 0; t < nv; ++t)
          for (int c = 0; c < 128; ++c) {
            double oi = 0.0, ci = 0.0;
            for (int d = 0; d < 128; ++d) oi += qf[t * 128 + d] * Hs[d * 128 + c];
            for (int s2 = 0; s2 < 64; ++s2) ci += AQ[t * 64 + s2] * vn[s2 * 128 + c];
            const double inter = (mutant == 1 ? oi : oi * eg[t]) * scale;
            const double r = ci * scale + inter;
            o[((bos + t0 + t) * HV + hv) * 128 + c] = exact ? f2bf((float)r) : f2bf((float)r);
          }
        const double dl = mutant == 3 ? 1.0 : std::exp2(glast);
        for (int d = 0; d < 128; ++d)
          for (int c = 0; c < 128; ++c) {
            double acc = h[d * 128 + c] * dl;
            for (int t = 0; t < 64; ++t) acc += kf[t * 128 + d] * vdec[t * 128 + c];
            h[d * 128 + c] = acc;
          }
      }
    }
  }
  return 0;
}

// Returns 0. units q/k: u < 2*KD/128 (q: u < KD/128); v: the rest. rstd_out (may be null): [Tf][2*KD/128].
// mutant != 0 plants a deliberate mistake (used only to show that the pinning tests catch it):
//   1: taps applied in reverse order (w[c][3 - j] with tap j)
//   2: a source row equal to meta.y taken from the cache instead of qkv
//   3: the L2 sum accumulated over the 128 channels in plain order
//   4: SiLU with the sign flipped inside the exponential
int oracle_conv(const uint16_t* qkv, long long SX, const uint16_t* cache, int C, const int* meta, const uint16_t* w,
                uint16_t* q, uint16_t* k, uint16_t* v, int Tf, float eps, int KD, int VD, int rep, int skip_v, int u0,
                int units, int mutant, float* rstd_out) {
  const int nqk = 2 * KD / 128, nq = KD / 128;
  for (int t = 0; t < Tf; ++t) {
    const int* m = meta + 4LL * t;
    for (int u = u0; u < u0 + units; ++u) {
      float s[128];
      for (int c = 0; c < 128; ++c) {
        const long long ch = 128LL * u + c;
        float acc = 0.f;
        for (int j = 0; j < 4; ++j) {
          const int src = m[0] - 3 + j;
          if (src < 0) continue;
          const bool from_qkv = mutant == 2 ? src > m[1] : src >= m[1];
          const uint16_t xb = from_qkv ? qkv[(long long)(m[2] + src) * SX + ch] : cache[(long long)(m[3] + src) * C + ch];
          const int jw = mutant == 1 ? 3 - j : j;
          acc = std::fmaf(bf2f(w[ch * 4 + jw]), bf2f(xb), acc);
        }
        const float y = bfr(acc);
        const float d = (float)(1.0 + std::exp(mutant == 4 ? (double)y : -(double)y));
        s[c] = bfr(y / d);
      }
      if (u < nqk) {
        float sum;
        if (mutant == 3) {
          sum = 0.f;
          for (int c = 0; c < 128; ++c) sum = std::fmaf(s[c], s[c], sum);
        } else {
          float g[16];
          for (int l = 0; l < 16; ++l) {
            const float* x = s + 8 * l;
            float p = x[1] * x[1];
            p = std::fmaf(x[0], x[0], p);
            for (int i = 2; i < 8; ++i) p = std::fmaf(x[i], x[i], p);
            g[l] = p;
          }
          for (int dist = 8; dist >= 1; dist >>= 1) {
            float h[16];
            for (int l = 0; l < 16; ++l) h[l] = g[l] + g[l ^ dist];
            for (int l = 0; l < 16; ++l) g[l] = h[l];
          }
          sum = g[0];
        }
        const float rstd = (float)(1.0 / std::sqrt((double)(eps + sum)));
        if (rstd_out) rstd_out[(long long)t * nqk + u] = rstd;
        const int REP = rep == 1 ? 1 : 2, nh = REP * KD / 128, hq = u % nq;
        uint16_t* dst = (u < nq ? q : k) + (long long)t * (nh * 128) + REP * hq * 128;
        for (int c = 0; c < 128; ++c) {
          dst[c] = f2bf(rstd * s[c]);
          if (REP == 2) dst[128 + c] = dst[c];
        }
      } else if (!skip_v) {
        uint16_t* dst = v + (long long)t * VD + (128LL * u - 2 * KD);
        for (int c = 0; c < 128; ++c) dst[c] = f2bf(s[c]);
      }
    }
  }
  return 0;
}

// mutant != 0 plants a deliberate mistake (used only to show that the pinning tests catch it):
//   1: decay 2^(g[c] - g[r]); 2: beta of the column; 3: the diagonal included in M; 4: the sign of the
//   off-diagonal entries lost (x_r = +sum)
int oracle_kkt(const uint16_t* k, const float* g, const uint16_t* beta, uint16_t* A, const int64_t* cu,
               const int64_t* cidx, int NT, int H, int HV, int mutant) {
  if (HV != 2 * H) return -1;
  for (int ch = 0; ch < NT; ++ch) {
    const int64_t i_n = cidx[2 * ch], i_t = cidx[2 * ch + 1];
    const int64_t bos = cu[i_n];
    const int T = (int)(cu[i_n + 1] - bos), t0 = (int)i_t * 64;
    const int nval = T - t0 < 64 ? T - t0 : 64;
    for (int kh = 0; kh < H; ++kh) {
      double raw[64][64];
      for (int r = 0; r < nval; ++r)
        for (int c = 0; c <= r; ++c) {
          double acc = 0.0;
          for (int d = 0; d < 128; ++d)
            acc += (double)bf2f(k[((bos + t0 + r) * H + kh) * 128 + d]) * (double)bf2f(k[((bos + t0 + c) * H + kh) * 128 + d]);
          raw[r][c] = acc;
        }
      for (int v = 0; v < 2; ++v) {
        const int hv = 2 * kh + v;
        auto G = [&](int r) { return g[(bos + t0 + r) * HV + hv]; };
        auto Bt = [&](int r) { return (double)bf2f(beta[(bos + t0 + r) * HV + hv]); };
        static thread_local double M[64][64];
        for (int r = 0; r < 64; ++r)
          for (int c = 0; c < 64; ++c) {
            M[r][c] = 0.0;
            const bool in = mutant == 3 ? c <= r : c < r;
            if (!in || r >= nval) continue;
            const float dg = mutant == 1 ? G(c) - G(r) : G(r) - G(c);
            M[r][c] = raw[r][c] * std::exp2((double)dg) * (mutant == 2 ? Bt(c) : Bt(r));
          }
        // X = (I + M)^-1, column by column
        double X[64][64];
        for (int j = 0; j < 64; ++j) {
          for (int r = 0; r < 64; ++r) {
            if (r < j) { X[r][j] = 0.0; continue; }
            double s = 0.0;
            for (int c = j; c < r; ++c) s += M[r][c] * X[c][j];
            if (mutant == 3) {
              X[r][j] = ((r == j ? 1.0 : 0.0) - s) / (1.0 + M[r][r]);
            } else {
              X[r][j] = r == j ? 1.0 : (mutant == 4 ? s : -s);
            }
          }
        }
        for (int r = 0; r < nval; ++r) {
          const int cend = 16 * (r / 16 + 1);
          for (int c = 0; c < cend; ++c) {
            const float xf = (float)X[r][c];
            A[((bos + t0 + r) * HV + hv) * 64 + c] = xf == 0.f ? 0 : f2bf(xf);
          }
        }
      }
    }
  }
  return 0;
}

}  // extern "C"
