// CPU oracle for the REAX fused-attention (FMHA) forward path.
//
// TEST INFRASTRUCTURE ONLY. This file is the checker, never the product: only tests/, the smoke check in
// __graft_entry__.py and the cpu_baseline leg of bench.py may load the library built from it.
//
// It restates, in plain C++, the math of the reference kernels
//   libreax_howu/reax_fmha_v8.cu        (fmha3_kernel + reax_fmha_b / reax_fmha_q)
//   libreax_fmha_post/reax_fmha_v11.cu  (the same kernel + the POST gate epilogue of reax_fmha_qp)
// as a direct two-pass softmax per query row, with the accumulation type a template parameter:
//   double : the correctness oracle;
//   float  : the OpenMP fp32 CPU baseline timed by bench.py (same source, same loops).
//
// Semantics restated (reference file:line):
//   - GQA row fold: row r of KV head h is query head h*G + r%G at token r/G          (v8:9, v8:147-148, v11:452)
//   - qpos mask: row r of batch b sees keys 0..qpos[b*qpBs + r/G]; qpos < 0 sees nothing   (v8:9-10, v8:276-277)
//   - bias mask: x = s*scale + bf16 bias[b][h][r][key], every key visible                (v8:279-280)
//   - logits: x = (s*scale + bias_or_0) in natural-log units; the kernel works in base 2  (v8:266-288)
//   - a row that sees no key, or whose visible logits are all -inf, outputs 0             (v8:303, v8:331-334)
//   - qpos = 0: the row sees key 0 only, so O = V[0] exactly                              (v8:224-235)
//   - drop-in block rule (reax_fmha_q / reax_fmha_qp only, Args::qpos0_block): folded rows of (b, h) form blocks
//     [64j, 64j + 64); when the largest raw qpos over a block's rows is 0, every row of the block, qpos < 0 rows
//     included, sees key 0 only and so stores V[0]                                        (v8:155-162, 224-235;
//                                                                                        v11:213-220, 282-293)
//   - POST: out[inv[b*Lq + r/G]][(h*G + r%G)*D + d] = bf16(bf16(o) * bf16(sigmoid(gate))), gate at +D in the
//     [T][Hq][2D] qg tensor; inv < 0 rows are skipped                                       (v11:451-522, 583-590)
// Extensions that the reference does not have (pinned only by this oracle and the tests that check it):
//   - LSE output: lse = log(sum_j exp(x_j)) over visible keys, -inf when nothing is visible;
//   - head_dim D as an argument (the reference fixes D = 256, v8:22);
//   - separate token / group strides for Q (row address b*qsB + h*qsH + (r/G)*qsT + (r%G)*qsG);
//   - varlen causal attention over packed sequences described by cu_seqlens;
//   - a key window [key_lo, key_hi) so that split-KV partials can be computed, and an LSE combine.
#pragma once
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <vector>

namespace oracle {

enum MaskMode : int32_t { MASK_QPOS = 0, MASK_BIAS = 1, MASK_VARLEN_CAUSAL = 2, MASK_NONE = 3 };

// Mirrors the arguments of reax_fmha_q / reax_fmha_b generalised as above. Strides are in elements.
struct Args {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const int32_t* qpos;
  const uint16_t* bias;
  const int32_t* cu_seqlens;
  int64_t qpBs;
  int64_t bsB, bsH, bsM;
  int64_t qsB, qsH, qsT, qsG;
  int64_t ksB, ksH, ksM;
  int64_t vsB, vsH, vsM;
  int32_t mask_mode;
  int32_t B, H, G, M, N, D;
  int32_t key_lo, key_hi;  // keys outside [key_lo, key_hi) are invisible; key_hi <= 0 means "no upper window"
  int32_t p_bf16;          // 1: round P to bf16 before P.V (the GPU kernels do), the row sum keeps fp P
  float scale;
  int32_t qpos0_block;     // 1: the drop-in entry points' block-wide qpos = 0 rule (see row_last_key)
};

// Deliberate mistakes that tests plant in the oracle (on the CPU) to show that the pins catch them.
enum Mutant : int32_t {
  MUT_NONE = 0,
  MUT_NO_SCALE = 1,        // logits not multiplied by scale
  MUT_GQA_HEAD_MAJOR = 2,  // row r read as head r / (M/G), token r % (M/G) instead of token r/G, head r%G
  MUT_CAUSAL_STRICT = 3,   // key j visible iff j < qpos instead of j <= qpos
  MUT_NO_NORMALISE = 4,    // O not divided by the row sum
  MUT_LSE_LOG2 = 5,        // LSE reported in base 2
  MUT_SIGMOID_SIGN = 6,    // sigmoid(-x)
  MUT_GATE_QUERY_HALF = 7, // POST reads the query half of qg (offset 0) instead of the gate half (offset D)
  MUT_COMBINE_NO_WEIGHT = 8,  // split combine averages partial outputs instead of LSE-weighting them
  MUT_BLOCK_TOKENS = 9,       // qpos = 0 block rule over blocks of 64 tokens instead of 64 folded rows
  MUT_BLOCK_CLAMPED = 10,     // qpos = 0 block rule on qpos clamped to N - 1 instead of the raw qpos
  MUT_BLOCK_OFF = 11,         // qpos = 0 block rule ignored (per-row rule only)
};
extern int32_t g_mutant;

inline float bf16_to_f32(uint16_t x) {
  const uint32_t u = (uint32_t)x << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// Correctly rounded (round-to-nearest-even) conversion of a double to bf16, without passing through fp32
// (double -> fp32 -> bf16 can round twice). Handles bf16 subnormals, overflow to inf and NaN.
inline uint16_t f64_to_bf16(double d) {
  if (std::isnan(d)) return 0x7fc0;
  const bool neg = std::signbit(d);
  const double a = std::fabs(d);
  double r;
  if (a == 0.0) {
    r = 0.0;
  } else if (a < std::ldexp(1.0, -126)) {
    r = std::ldexp(std::nearbyint(std::ldexp(a, 133)), -133);  // subnormal spacing 2^-133
  } else {
    int e;
    const double m = std::frexp(a, &e);  // a = m * 2^e, m in [0.5, 1)
    r = std::ldexp(std::nearbyint(std::ldexp(m, 8)), e - 8);  // 8 significant bits
  }
  uint16_t bits;
  if (r >= std::ldexp(1.0, 128)) {
    bits = 0x7f80;  // overflow rounds to infinity
  } else {
    const float f = (float)r;  // exact: r has at most 8 significant bits and is in fp32 range
    uint32_t u;
    std::memcpy(&u, &f, 4);
    bits = (uint16_t)(u >> 16);
  }
  return (uint16_t)(bits | (neg ? 0x8000 : 0));
}

inline uint16_t f32_to_bf16(float f) { return f64_to_bf16((double)f); }

// Correctly rounded bf16 sigmoid of a bf16 gate value (evaluated in double).
inline uint16_t sigmoid_bf16(uint16_t x) {
  double g = (double)bf16_to_f32(x);
  if (g_mutant == MUT_SIGMOID_SIGN) g = -g;
  if (std::isnan(g)) return 0x7fc0;
  const double s = g >= 0 ? 1.0 / (1.0 + std::exp(-g)) : std::exp(g) / (1.0 + std::exp(g));
  return f64_to_bf16(s);
}

template <typename T>
inline T exp_t(T x) { return std::exp(x); }
template <typename T>
inline T log_t(T x) { return std::log(x); }

// Per-batch geometry: varlen packs sequences along the token axis, otherwise every batch has M rows, N keys.
struct BatchView {
  int64_t tok0;  // first token of this batch entry on the token axis (varlen), else 0
  int32_t rows;  // valid rows (folded: tokens * G)
  int32_t keys;  // keys
};

inline BatchView batch_view(const Args& a, int b) {
  if (a.mask_mode == MASK_VARLEN_CAUSAL) {
    const int32_t s0 = a.cu_seqlens[b], s1 = a.cu_seqlens[b + 1];
    return BatchView{s0, (s1 - s0) * a.G, s1 - s0};
  }
  return BatchView{0, a.M, a.N};
}

// Largest qpos over the 64-row block of folded row r (reax_fmha_v8.cu:141-162: cta_qmax over the CTA's 64 rows,
// rows at or beyond M count as -1). The reference compares the raw qpos, before any clamp to the key count.
inline int64_t block_qpos_max(const Args& a, int b, int r, const BatchView& bv) {
  const int64_t M = bv.rows;
  int64_t lo, hi;  // row range [lo, hi) of the block
  if (g_mutant == MUT_BLOCK_TOKENS) {
    const int64_t t0 = (int64_t)(r / a.G) / 64 * 64;
    lo = t0 * a.G;
    hi = lo + 64LL * a.G;
  } else {
    lo = (int64_t)r / 64 * 64;
    hi = lo + 64;
  }
  if (hi > M) hi = M;
  int64_t mx = -1;
  for (int64_t rr = lo; rr < hi; ++rr) {
    int64_t qp = a.qpos[(int64_t)b * a.qpBs + rr / a.G];
    if (g_mutant == MUT_BLOCK_CLAMPED && qp > bv.keys - 1) qp = bv.keys - 1;
    if (qp > mx) mx = qp;
  }
  return mx;
}

// Last key index (inclusive) that row r may see before the key window, or -1.
inline int64_t row_last_key(const Args& a, int b, int r, const BatchView& bv) {
  const int tok = r / a.G;
  switch (a.mask_mode) {
    case MASK_QPOS: {
      if (a.qpos0_block && g_mutant != MUT_BLOCK_OFF && bv.keys > 0 && block_qpos_max(a, b, r, bv) == 0) return 0;
      const int64_t qp = a.qpos[(int64_t)b * a.qpBs + tok];
      if (qp < 0) return -1;
      const int64_t lim = g_mutant == MUT_CAUSAL_STRICT ? qp - 1 : qp;
      return lim < bv.keys - 1 ? lim : bv.keys - 1;
    }
    case MASK_VARLEN_CAUSAL: {
      const int64_t lim = g_mutant == MUT_CAUSAL_STRICT ? tok - 1 : tok;
      return lim < bv.keys - 1 ? lim : bv.keys - 1;
    }
    default:
      return bv.keys - 1;
  }
}

// One output row: o[0..D) and *lse. Acc is the accumulation type (double oracle / float baseline).
template <typename Acc>
void attn_row(const Args& a, int b, int h, int r, const BatchView& bv, Acc* o, Acc* lse, std::vector<Acc>& qrow,
              std::vector<Acc>& x) {
  const int D = a.D;
  const int Mtok = a.M / a.G > 0 ? a.M / a.G : 1;
  int tok = r / a.G, g = r % a.G;
  if (g_mutant == MUT_GQA_HEAD_MAJOR && a.mask_mode != MASK_VARLEN_CAUSAL) {
    g = r / Mtok;
    tok = r % Mtok;
    if (g >= a.G) g = a.G - 1;
  }
  const uint16_t* qp = a.q + (int64_t)b * a.qsB + (int64_t)h * a.qsH + (bv.tok0 + tok) * a.qsT + (int64_t)g * a.qsG;
  const uint16_t* kb = a.k + (int64_t)b * a.ksB + (int64_t)h * a.ksH + bv.tok0 * a.ksM;
  const uint16_t* vb = a.v + (int64_t)b * a.vsB + (int64_t)h * a.vsH + bv.tok0 * a.vsM;
  for (int d = 0; d < D; ++d) qrow[d] = (Acc)bf16_to_f32(qp[d]);

  int64_t hi = row_last_key(a, b, r, bv);  // inclusive
  int64_t lo = 0;
  if (a.key_lo > lo) lo = a.key_lo;
  if (a.key_hi > 0 && a.key_hi - 1 < hi) hi = a.key_hi - 1;

  const Acc scale = g_mutant == MUT_NO_SCALE ? (Acc)1 : (Acc)a.scale;
  const Acc ninf = -std::numeric_limits<Acc>::infinity();
  Acc mx = ninf;
  for (int64_t j = lo; j <= hi; ++j) {
    const uint16_t* kr = kb + j * a.ksM;
    Acc s = 0;
#pragma omp simd reduction(+ : s)
    for (int d = 0; d < D; ++d) s += qrow[d] * (Acc)bf16_to_f32(kr[d]);
    Acc xv = s * scale;
    if (a.mask_mode == MASK_BIAS) {
      const uint16_t* br = a.bias + (int64_t)b * a.bsB + (int64_t)h * a.bsH + (int64_t)r * a.bsM;
      xv += (Acc)bf16_to_f32(br[j]);
    }
    x[j - lo] = xv;
    if (xv > mx) mx = xv;
  }
  for (int d = 0; d < D; ++d) o[d] = 0;
  if (hi < lo || mx == ninf) {  // nothing visible (or every visible logit is -inf): O = 0, LSE = -inf
    *lse = ninf;
    return;
  }
  Acc l = 0;
  for (int64_t j = lo; j <= hi; ++j) {
    const Acc p = exp_t<Acc>(x[j - lo] - mx);
    l += p;
    const Acc w = a.p_bf16 ? (Acc)bf16_to_f32(f64_to_bf16((double)p)) : p;
    if (w == 0) continue;
    const uint16_t* vr = vb + j * a.vsM;
#pragma omp simd
    for (int d = 0; d < D; ++d) o[d] += w * (Acc)bf16_to_f32(vr[d]);
  }
  if (g_mutant != MUT_NO_NORMALISE) {
    for (int d = 0; d < D; ++d) o[d] /= l;
  }
  Acc lv = mx + log_t<Acc>(l);
  if (g_mutant == MUT_LSE_LOG2) lv = lv / (Acc)0.69314718055994530942;
  *lse = lv;
}

// Whole problem, rows of every (b, h). Output is dense: o[((b*H + h)*Mo + r)*D + d], lse[(b*H + h)*Mo + r],
// Mo = a.M (for varlen a.M is the largest rows-per-sequence). If rows != nullptr only those row indices
// are computed (for every b, h); other entries are left untouched.
template <typename Acc>
void attn(const Args& a, Acc* o, Acc* lse, const int32_t* rows, int nrows, int nthreads) {
  const int D = a.D, Mo = a.M;
  const int64_t nr = rows ? nrows : Mo;
  const int64_t total = (int64_t)a.B * a.H * nr;
  int maxkeys = a.N;
  if (a.mask_mode == MASK_VARLEN_CAUSAL)
    for (int b = 0; b < a.B; ++b) maxkeys = std::max(maxkeys, a.cu_seqlens[b + 1] - a.cu_seqlens[b]);
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1)
  {
    std::vector<Acc> qrow(D), x(maxkeys > 0 ? maxkeys : 1);
#pragma omp for schedule(dynamic, 4)
    for (int64_t i = 0; i < total; ++i) {
      const int b = (int)(i / ((int64_t)a.H * nr));
      const int h = (int)((i / nr) % a.H);
      const int r = rows ? rows[i % nr] : (int)(i % nr);
      const BatchView bv = batch_view(a, b);
      if (r < 0 || r >= bv.rows || r >= Mo) continue;
      const int64_t orow = ((int64_t)b * a.H + h) * Mo + r;
      attn_row<Acc>(a, b, h, r, bv, o + orow * D, lse + orow, qrow, x);
    }
  }
}

// LSE-weighted merge of S partial results for R rows: part_o[(s*R + r)*D + d], part_lse[s*R + r].
inline void lse_combine(const double* part_o, const double* part_lse, int S, int R, int D, double* o, double* lse) {
  for (int r = 0; r < R; ++r) {
    double mx = -std::numeric_limits<double>::infinity();
    for (int s = 0; s < S; ++s) mx = std::max(mx, part_lse[(int64_t)s * R + r]);
    double* orow = o + (int64_t)r * D;
    for (int d = 0; d < D; ++d) orow[d] = 0;
    if (mx == -std::numeric_limits<double>::infinity()) {
      lse[r] = mx;
      continue;
    }
    double wsum = 0;
    for (int s = 0; s < S; ++s) wsum += std::exp(part_lse[(int64_t)s * R + r] - mx);
    for (int s = 0; s < S; ++s) {
      const double ls = part_lse[(int64_t)s * R + r];
      double w = std::exp(ls - mx) / wsum;
      if (g_mutant == MUT_COMBINE_NO_WEIGHT) w = ls == -std::numeric_limits<double>::infinity() ? 0.0 : 1.0 / S;
      for (int d = 0; d < D; ++d) orow[d] += w * part_o[((int64_t)s * R + r) * D + d];
    }
    lse[r] = mx + std::log(wsum);
  }
}

}  // namespace oracle
