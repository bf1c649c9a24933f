// extern "C" entry points of libreax_howu.so (REAX_LIB_HOWU) and libreax_fmha_post.so (REAX_LIB_POST).
// The prototypes are those of the reference (libreax_howu/reax_fmha_v8.cu:434-450,
// libreax_fmha_post/reax_fmha_v11.cu:565-590) plus the extension entry points declared in include/.
// Each one fills a FwdParams block and launches asynchronously on the caller's stream; nothing is allocated,
// cached or synchronised here.
#include <hip/hip_runtime.h>

#include "fmha_launch.h"

#pragma GCC visibility push(default)
#if defined(REAX_LIB_POST)
#include "libreax_fmha_post.h"
#else
#include "libreax_howu.h"
#endif
#pragma GCC visibility pop

using reax::FwdParams;

namespace {

FwdParams base_params(const void* q, const void* k, const void* v, void* o, float scale, int B, int H, int M, int N) {
  FwdParams p{};
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.o = static_cast<uint16_t*>(o);
  p.scale = scale;
  p.B = B;
  p.H = H;
  p.M = M;
  p.N = N;
  p.G = 1;
  return p;
}

void set_kv(FwdParams& p, long long ksB, long long ksH, long long ksM, long long vsB, long long vsH, long long vsM) {
  p.ksB = ksB;
  p.ksH = ksH;
  p.ksM = ksM;
  p.vsB = vsB;
  p.vsH = vsH;
  p.vsM = vsM;
}

}  // namespace

extern "C" {

// bias mode (reax_fmha_v8.cu:434-442): every key visible, x = s*scale + bias; NULL bias -> -1
int reax_fmha_b(const void* q, const void* k, const void* v, const void* bias, void* o, float scale, int B, int H,
                int M, int N, long long qsB, long long qsH, long long qsM, long long ksB, long long ksH, long long ksM,
                long long vsB, long long vsH, long long vsM, long long bsB, long long bsH, long long bsM,
                long long osB, long long osH, long long osM, void* stream) {
  if (!bias) return -1;
  FwdParams p = base_params(q, k, v, o, scale, B, H, M, N);
  p.bias = static_cast<const uint16_t*>(bias);
  p.bsB = bsB;
  p.bsH = bsH;
  p.bsM = bsM;
  p.qsB = qsB;
  p.qsH = qsH;
  p.qsT = qsM;
  p.qsG = 0;
  set_kv(p, ksB, ksH, ksM, vsB, vsH, vsM);
  p.osB = osB;
  p.osH = osH;
  p.osT = osM;
  p.osG = 0;
  return reax::launch_fwd(p, 256, reax::MODE_BIAS, false, static_cast<hipStream_t>(stream));
}

// qpos mode (reax_fmha_v8.cu:443-450): row r sees keys 0..qpos[b*qpBs + r/G]; row r at r*qsM = (r/G)*(G*qsM) + (r%G)*qsM.
// A 64-row block whose largest qpos is 0 stores V[0] in every row, qpos < 0 rows included (v8:155-162, 224-235).
int reax_fmha_q(const void* q, const void* k, const void* v, const int* qpos, int G, long long qpBs, void* o,
                float scale, int B, int H, int M, int N, long long qsB, long long qsH, long long qsM, long long ksB,
                long long ksH, long long ksM, long long vsB, long long vsH, long long vsM, long long osB, long long osH,
                long long osM, void* stream) {
  if (!qpos) return (int)hipErrorInvalidValue;
  FwdParams p = base_params(q, k, v, o, scale, B, H, M, N);
  p.qpos = qpos;
  p.qpBs = qpBs;
  p.G = G;
  p.qsB = qsB;
  p.qsH = qsH;
  p.qsT = (long long)G * qsM;
  p.qsG = qsM;
  set_kv(p, ksB, ksH, ksM, vsB, vsH, vsM);
  p.osB = osB;
  p.osH = osH;
  p.osT = (long long)G * osM;
  p.osG = osM;
  p.qpos0_block = 1;
  return reax::launch_fwd(p, 256, reax::MODE_QPOS, false, static_cast<hipStream_t>(stream));
}

#if defined(REAX_LIB_POST)

// qpos mode + attn_post epilogue (reax_fmha_v11.cu:583-590)
int reax_fmha_qp(const void* q, const void* k, const void* v, const int* qpos, int G, long long qpBs, float scale,
                 int B, int H, int M, int N, long long qsB, long long qsH, long long qsM, long long ksB, long long ksH,
                 long long ksM, long long vsB, long long vsH, long long vsM, const int* inv, int Lq, const void* qg,
                 long long qg_rs, void* outp, long long out_rs, void* stream) {
  if (!qpos) return (int)hipErrorInvalidValue;
  FwdParams p = base_params(q, k, v, nullptr, scale, B, H, M, N);
  p.qpos = qpos;
  p.qpBs = qpBs;
  p.G = G;
  p.qsB = qsB;
  p.qsH = qsH;
  p.qsT = (long long)G * qsM;
  p.qsG = qsM;
  set_kv(p, ksB, ksH, ksM, vsB, vsH, vsM);
  p.inv = inv;
  p.Lq = Lq;
  p.qg = static_cast<const uint16_t*>(qg);
  p.qg_rs = qg_rs;
  p.outp = static_cast<uint16_t*>(outp);
  p.out_rs = out_rs;
  p.qpos0_block = 1;
  return reax::launch_fwd(p, 256, reax::MODE_QPOS, true, static_cast<hipStream_t>(stream));
}

#else  // libreax_howu.so: extension entry points

int reax_fmha_qx(const void* q, const void* k, const void* v, const int* qpos, int G, long long qpBs, void* o,
                 float* lse, float scale, int B, int H, int M, int N, int D, long long qsB, long long qsH,
                 long long qsT, long long qsG, long long ksB, long long ksH, long long ksM, long long vsB,
                 long long vsH, long long vsM, long long osB, long long osH, long long osT, long long osG,
                 long long lsB, long long lsH, long long lsT, long long lsG, void* stream) {
  if (!qpos) return (int)hipErrorInvalidValue;
  FwdParams p = base_params(q, k, v, o, scale, B, H, M, N);
  p.qpos = qpos;
  p.qpBs = qpBs;
  p.G = G;
  p.lse = lse;
  p.qsB = qsB;
  p.qsH = qsH;
  p.qsT = qsT;
  p.qsG = qsG;
  set_kv(p, ksB, ksH, ksM, vsB, vsH, vsM);
  p.osB = osB;
  p.osH = osH;
  p.osT = osT;
  p.osG = osG;
  p.lsB = lsB;
  p.lsH = lsH;
  p.lsT = lsT;
  p.lsG = lsG;
  return reax::launch_fwd(p, D, reax::MODE_QPOS, false, static_cast<hipStream_t>(stream));
}

int reax_fmha_varlen(const void* q, const void* k, const void* v, const int* cu_seqlens, int nseq, int max_seqlen,
                     void* o, float* lse, float scale, int Hq, int Hkv, int D, long long qsT, long long qsH,
                     long long ksT, long long ksH, long long vsT, long long vsH, long long osT, long long osH,
                     long long lsT, long long lsH, void* stream) {
  if (!cu_seqlens || Hkv <= 0 || Hq <= 0 || Hq % Hkv != 0 || max_seqlen < 0) return (int)hipErrorInvalidValue;
  const int G = Hq / Hkv;
  FwdParams p = base_params(q, k, v, o, scale, nseq, Hkv, (int)((long long)max_seqlen * G), max_seqlen);
  if ((long long)max_seqlen * G > 0x7fffffffLL) return (int)hipErrorInvalidValue;
  p.cu_seqlens = cu_seqlens;
  p.G = G;
  p.lse = lse;
  p.qsB = 0;
  p.qsH = (long long)G * qsH;
  p.qsT = qsT;
  p.qsG = qsH;
  set_kv(p, 0, ksH, ksT, 0, vsH, vsT);
  p.osB = 0;
  p.osH = (long long)G * osH;
  p.osT = osT;
  p.osG = osH;
  p.lsB = 0;
  p.lsH = (long long)G * lsH;
  p.lsT = lsT;
  p.lsG = lsH;
  return reax::launch_fwd(p, D, reax::MODE_VARLEN, false, static_cast<hipStream_t>(stream));
}

size_t reax_fmha_splitkv_workspace(int B, int H, int M, int D, int num_splits) {
  return reax::splitkv_workspace_bytes(B, H, M, D, num_splits);
}

int reax_fmha_splitkv(const void* q, const void* k, const void* v, const int* qpos, int G, long long qpBs, void* o,
                      float* lse, float scale, int B, int H, int M, int N, int D, int num_splits, void* ws,
                      size_t ws_bytes, long long qsB, long long qsH, long long qsT, long long qsG, long long ksB,
                      long long ksH, long long ksM, long long vsB, long long vsH, long long vsM, long long osB,
                      long long osH, long long osT, long long osG, long long lsB, long long lsH, long long lsT,
                      long long lsG, void* stream) {
  if (!qpos) return (int)hipErrorInvalidValue;
  reax::SplitParams sp{};
  FwdParams& p = sp.f;
  p = base_params(q, k, v, o, scale, B, H, M, N);
  p.qpos = qpos;
  p.qpBs = qpBs;
  p.G = G;
  p.lse = lse;
  p.qsB = qsB;
  p.qsH = qsH;
  p.qsT = qsT;
  p.qsG = qsG;
  set_kv(p, ksB, ksH, ksM, vsB, vsH, vsM);
  p.osB = osB;
  p.osH = osH;
  p.osT = osT;
  p.osG = osG;
  p.lsB = lsB;
  p.lsH = lsH;
  p.lsT = lsT;
  p.lsG = lsG;
  sp.num_splits = num_splits;
  sp.ws = ws;
  sp.ws_bytes = ws_bytes;
  return reax::launch_splitkv(sp, D, static_cast<hipStream_t>(stream));
}

int reax_fmha_splitkv_noalloc(const void* q, const void* k, const void* v, const int* qpos, int G, long long qpBs,
                              void* o, float* lse, float scale, int B, int H, int M, int N, int D, int num_splits,
                              long long qsB, long long qsH, long long qsT, long long qsG, long long ksB,
                              long long ksH, long long ksM, long long vsB, long long vsH, long long vsM,
                              long long osB, long long osH, long long osT, long long osG, long long lsB,
                              long long lsH, long long lsT, long long lsG, void* stream) {
  if (!qpos) return (int)hipErrorInvalidValue;
  reax::SplitParams sp{};
  FwdParams& p = sp.f;
  p = base_params(q, k, v, o, scale, B, H, M, N);
  p.qpos = qpos;
  p.qpBs = qpBs;
  p.G = G;
  p.lse = lse;
  p.qsB = qsB;
  p.qsH = qsH;
  p.qsT = qsT;
  p.qsG = qsG;
  set_kv(p, ksB, ksH, ksM, vsB, vsH, vsM);
  p.osB = osB;
  p.osH = osH;
  p.osT = osT;
  p.osG = osG;
  p.lsB = lsB;
  p.lsH = lsH;
  p.lsT = lsT;
  p.lsG = lsG;
  sp.num_splits = num_splits;
  return reax::launch_splitkv_noalloc(sp, D, static_cast<hipStream_t>(stream));
}

#endif

}  // extern "C"
