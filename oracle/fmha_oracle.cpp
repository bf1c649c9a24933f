// C entry points of the CPU oracle (ctypes-friendly). TEST INFRASTRUCTURE ONLY: see fmha_oracle.h.
#include "fmha_oracle.h"

#include <algorithm>

namespace oracle {
int32_t g_mutant = MUT_NONE;
}

using namespace oracle;

extern "C" {

void oracle_set_mutant(int32_t m) { g_mutant = m; }
int32_t oracle_get_mutant() { return g_mutant; }

// Double-precision oracle (see attn<> for the output layout). Returns 0, or -1 on bad arguments.
int oracle_attn_f64(const Args* a, double* o, double* lse, const int32_t* rows, int32_t nrows, int32_t nthreads) {
  if (!a || !o || !lse || a->D <= 0 || a->G <= 0 || a->B < 0 || a->H < 0) return -1;
  attn<double>(*a, o, lse, rows, nrows, nthreads);
  return 0;
}

// The same math accumulated in fp32: the OpenMP CPU baseline.
int oracle_attn_f32(const Args* a, float* o, float* lse, const int32_t* rows, int32_t nrows, int32_t nthreads) {
  if (!a || !o || !lse || a->D <= 0 || a->G <= 0 || a->B < 0 || a->H < 0) return -1;
  attn<float>(*a, o, lse, rows, nrows, nthreads);
  return 0;
}

uint16_t oracle_f64_to_bf16(double d) { return f64_to_bf16(d); }

void oracle_f64_to_bf16_array(const double* x, uint16_t* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = f64_to_bf16(x[i]);
}

uint16_t oracle_sigmoid_bf16(uint16_t x) { return sigmoid_bf16(x); }

// All 65,536 bf16 inputs: out[x] = bf16(sigmoid(bf16 x)), correctly rounded.
void oracle_sigmoid_bf16_all(uint16_t* out) {
  for (uint32_t x = 0; x < 65536u; ++x) out[x] = sigmoid_bf16((uint16_t)x);
}

// POST epilogue of reax_fmha_qp (v11:451-522): o is the dense oracle output [B][H][M][D] (double); rows
// r < M of (b, h) with R = inv[b*Lq + r/G] >= 0 write
//   out[R*out_rs + (h*G + r%G)*D + d] = bf16(bf16(o) * bf16(sigmoid(qg[R*qg_rs + (h*G + r%G)*2D + D + d])))
// where the bf16 x bf16 product is rounded once (it is exact in double). Rows with R < 0 are not written.
int oracle_post_gate(const double* o, int32_t B, int32_t H, int32_t G, int32_t M, int32_t D, const int32_t* inv,
                     int32_t Lq, const uint16_t* qg, int64_t qg_rs, uint16_t* out, int64_t out_rs) {
  if (!o || !inv || !qg || !out || G <= 0 || D <= 0) return -1;
  const int64_t gate_off = g_mutant == MUT_GATE_QUERY_HALF ? 0 : D;
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h)
      for (int r = 0; r < M; ++r) {
        const int32_t R = inv[(int64_t)b * Lq + r / G];
        if (R < 0) continue;
        const int64_t hq = (int64_t)h * G + r % G;
        const double* orow = o + (((int64_t)b * H + h) * M + r) * D;
        const uint16_t* grow = qg + (int64_t)R * qg_rs + hq * 2 * D + gate_off;
        uint16_t* dst = out + (int64_t)R * out_rs + hq * D;
        for (int d = 0; d < D; ++d) {
          const double ob = (double)bf16_to_f32(f64_to_bf16(orow[d]));
          const double sg = (double)bf16_to_f32(sigmoid_bf16(grow[d]));
          dst[d] = f64_to_bf16(ob * sg);
        }
      }
  return 0;
}

// LSE-weighted combine of split partials (see lse_combine).
int oracle_lse_combine(const double* part_o, const double* part_lse, int32_t S, int32_t R, int32_t D, double* o,
                       double* lse) {
  if (!part_o || !part_lse || !o || !lse || S <= 0) return -1;
  lse_combine(part_o, part_lse, S, R, D, o, lse);
  return 0;
}

int32_t oracle_args_size() { return (int32_t)sizeof(Args); }

}  // extern "C"
