/* C ABI of libreax_howu.so, the MI355X (gfx950) rebuild of the reference's howu library.
 *
 * Conventions (as in the reference, libreax_howu/reax_fmha_v8.cu:434-450): caller-owned device pointers, the
 * library allocates nothing (the split-KV entry takes a caller workspace), strides in elements, head-dim
 * stride 1, asynchronous on `stream` (hipStream_t, NULL = default stream), return 0 or a hipError_t code.
 * H is the KV-head count; folded row r of KV head h is query head h*G + r%G at token r/G.
 *
 * Three groups of symbols:
 *   1. the reference's FMHA entry points (drop-in, head_dim 256);
 *   2. extension entry points for what the reference ABI cannot express (head_dim 128, LSE output, two-stride
 *      [S][Hq][D] row addressing, packed varlen sequences, split-KV decode with an LSE combine);
 *   3. the reference's other kernels of this library: reduce-add RMSNorm (reax_rarn), causal conv + SiLU + L2 norm
 *      (reax_conv_l2, reax_conv_v), Gated-DeltaNet chunk solve (reax_kkt, reax_kkt_smem) and chunked forward
 *      (reax_howu, howu3_skip, howu3_dense, howu3_smem, reax_howu_norm).
 */
#ifndef LIBREAX_HOWU_H
#define LIBREAX_HOWU_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif


/* ---- 1. reference FMHA entry points ------------------------------------------------------------------- */

/* Additive-bias attention. Replaces reax_fmha_b, libreax_howu/reax_fmha_v8.cu:434-442. */
int reax_fmha_b(const void* q, const void* k, const void* v, const void* bias, void* o, float scale, int B, int H,
                int M, int N, long long qsB, long long qsH, long long qsM, long long ksB, long long ksH, long long ksM,
                long long vsB, long long vsH, long long vsM, long long bsB, long long bsH, long long bsM,
                long long osB, long long osH, long long osM, void* stream);

/* qpos / causal GQA attention. Replaces reax_fmha_q, libreax_howu/reax_fmha_v8.cu:443-450. */
int reax_fmha_q(const void* q, const void* k, const void* v, const int* qpos, int G, long long qpBs, void* o,
                float scale, int B, int H, int M, int N, long long qsB, long long qsH, long long qsM, long long ksB,
                long long ksH, long long ksM, long long vsB, long long vsH, long long vsM, long long osB, long long osH,
                long long osM, void* stream);

/* ---- 2. extension entry points (no counterpart in the reference) --------------------------------------- */

/* reax_fmha_q generalised (extends libreax_howu/reax_fmha_v8.cu:443-450):
 *   - D in {128, 256};
 *   - row r of (b, h) is read at q + b*qsB + h*qsH + (r/G)*qsT + (r%G)*qsG (reax_fmha_q is qsT = G*qsM,
 *     qsG = qsM); for [B][S][Hq][D] tensors: qsB = S*Hq*D, qsH = G*D, qsT = Hq*D, qsG = D; O likewise;
 *   - lse (optional, fp32): natural-log logsumexp of the scaled logits of each row, -inf for a row that sees
 *     no key, written at lse + b*lsB + h*lsH + (r/G)*lsT + (r%G)*lsG. */
int reax_fmha_qx(const void* q, const void* k, const void* v, const int* qpos, int G, long long qpBs, void* o,
                 float* lse, float scale, int B, int H, int M, int N, int D, long long qsB, long long qsH,
                 long long qsT, long long qsG, long long ksB, long long ksH, long long ksM, long long vsB,
                 long long vsH, long long vsM, long long osB, long long osH, long long osT, long long osG,
                 long long lsB, long long lsH, long long lsT, long long lsG, void* stream);

/* Packed variable-length causal attention. Sequence b occupies tokens cu_seqlens[b] .. cu_seqlens[b+1]-1 of
 * Q/O [T][Hq][D] and K/V [T][Hkv][D] (token strides qsT/ksT/vsT/osT, head strides qsH/ksH/vsH/osH); token i of
 * a sequence sees that sequence's tokens 0..i only. cu_seqlens (int32, nseq+1 entries, device memory) starts at
 * 0 and is non-decreasing; max_seqlen >= every sequence length. lse (optional) is [T][Hq] with strides
 * lsT/lsH. Hq must be a multiple of Hkv. max_seqlen sizes the launch and cu_seqlens is device memory the host
 * does not read, so a max_seqlen below some sequence's length is not detected: that sequence's tokens past
 * max_seqlen may be left unwritten in o and lse (flash-attention's varlen interface has the same precondition). */
int reax_fmha_varlen(const void* q, const void* k, const void* v, const int* cu_seqlens, int nseq, int max_seqlen,
                     void* o, float* lse, float scale, int Hq, int Hkv, int D, long long qsT, long long qsH,
                     long long ksT, long long ksH, long long vsT, long long vsH, long long osT, long long osH,
                     long long lsT, long long lsH, void* stream);

/* Bytes of device workspace reax_fmha_splitkv needs (0 for unsupported arguments). */
size_t reax_fmha_splitkv_workspace(int B, int H, int M, int D, int num_splits);

/* Split-KV attention for short query blocks (decode): same arguments and result as reax_fmha_qx, computed as
 * num_splits independent key ranges (partial O and LSE in `ws`) merged by an LSE-weighted combine kernel.
 * ws: device memory, 256-byte aligned, at least reax_fmha_splitkv_workspace(...) bytes, owned by the caller;
 * it is overwritten, and calls that share it must be ordered on one stream. */
int reax_fmha_splitkv(const void* q, const void* k, const void* v, const int* qpos, int G, long long qpBs, void* o,
                      float* lse, float scale, int B, int H, int M, int N, int D, int num_splits, void* ws,
                      size_t ws_bytes, long long qsB, long long qsH, long long qsT, long long qsG, long long ksB,
                      long long ksH, long long ksM, long long vsB, long long vsH, long long vsM, long long osB,
                      long long osH, long long osT, long long osG, long long lsB, long long lsH, long long lsT,
                      long long lsG, void* stream);

/* reax_fmha_splitkv without a workspace argument, for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc); it has no counterpart in the reference. The partials go
 * to a static device array of 8 MiB that each GPU the library runs on holds until the process ends; nothing on the
 * call path allocates. Same arguments (minus ws / ws_bytes), kernels and result as reax_fmha_splitkv. Returns
 * hipErrorOutOfMemory (2) when reax_fmha_splitkv_workspace(B, H, M, D, num_splits) exceeds 8 MiB (config 4, B 16,
 * 8 KV heads, 4 rows, 16 splits, needs 4.2 MB). Every call on one GPU shares that GPU's array: calls that overlap
 * on one GPU race (order them on one stream). */
int reax_fmha_splitkv_noalloc(const void* q, const void* k, const void* v, const int* qpos, int G, long long qpBs,
                              void* o, float* lse, float scale, int B, int H, int M, int N, int D, int num_splits,
                              long long qsB, long long qsH, long long qsT, long long qsG, long long ksB,
                              long long ksH, long long ksM, long long vsB, long long vsH, long long vsM,
                              long long osB, long long osH, long long osT, long long osG, long long lsB,
                              long long lsH, long long lsT, long long lsG, void* stream);

/* ---- 3. the reference's Gated-DeltaNet / norm / conv entry points ------------------------------------------ */

/* Reduce-add RMSNorm. Replaces reax_rarn, libreax_howu/reax_rarn_final.cu:98-106. Rows of D = 2560 bf16:
 * h = bf16(res + bf16(part[0] + ... + part[S-1])) (serial != 0: rounded to bf16 after every add), written to h_out;
 * out = bf16(h * r * (1 + w)) with r = 1/sqrt(factor * sum(h^2) + eps), the sum in the reference's fixed order.
 * part: S partials, pstride elements apart. Returns 0 for n <= 0, -1 for D != 2560, -2 for S outside 2..8 (the
 * reference's codes), hipErrorInvalidValue for a null buffer or rows not 4-byte aligned, else hipGetLastError().
 * r is computed in double precision and rounded to fp32, where the reference uses the approximate rsqrtf. */
int reax_rarn(const void* part, int S, int serial, long long pstride, const void* res, const void* w, void* h_out,
              void* out, int n, int D, float eps, float factor, void* stream);

/* Causal 4-tap conv1d + SiLU + per-head L2 norm of q/k. Replaces reax_conv_l2, libreax_howu/reax_conv_v2.cu:164-181.
 * Token t (meta[t] = {position, first position held by qkv, qkv row offset, cache row offset}) reads source
 * positions position-3 .. position (skipping negative ones) from qkv (row stride SX) or the conv cache (row stride
 * C); channels form 128-wide units: KD/128 q heads, KD/128 k heads, then VD/128 v heads; w is [2*KD + VD][4] bf16.
 * q/k: bf16(s * rstd) with rstd = 1/sqrt(eps + sum of s^2 over the head), written once (rep 1) or twice side by side
 * (rep != 1) into q/k rows of rep*KD; v (unless skip_v): s, rows of VD. s = bf16(y / (1 + exp(-y))), y = bf16(conv).
 * Returns 0 for Tf <= 0, -1 for RT outside {8, 16, 32} (the reference's codes; RT is its tiling choice and only
 * checked here), hipErrorInvalidValue for missing buffers, KD not a positive multiple of 128, VD not a multiple of
 * 128, or rows / meta / outputs not 16-byte aligned, weights not 8-byte aligned; else hipGetLastError(). qkv must
 * hold at least one row. exp and 1/sqrt are evaluated to fp32 accuracy where the reference uses CUDA's fast
 * approximations: a bf16 result can differ from the reference's by one ulp in rare elements. */
int reax_conv_l2(const void* qkv, long long SX, const void* cache, int C, const void* meta, const void* w, void* q,
                 void* k, void* v, int Tf, float eps, int KD, int VD, int rep, int skip_v, int RT, void* stream);
/* The value units only (v = s, no q/k outputs). Replaces reax_conv_v, libreax_howu/reax_conv_v2.cu:183-189.
 * Returns 0 for Tf <= 0, hipErrorInvalidValue as reax_conv_l2, else hipGetLastError(). */
int reax_conv_v(const void* qkv, long long SX, const void* cache, int C, const void* meta, const void* w, void* v,
                int Tf, int KD, int VD, void* stream);

/* Gated-DeltaNet chunk solve. Replaces reax_kkt, libreax_howu/reax_kkt.cu:263-271. For chunk n (cidx[2n] = sequence,
 * cidx[2n+1] = 64-token chunk of it; cu = int64 sequence starts) and key head kh, for value heads hv = 2kh, 2kh+1:
 * A = (I + M)^-1 with M[r][c] = (k_r . k_c) * 2^(g[r] - g[c]) * beta[r] for c < r within the chunk; k bf16
 * [T][H][128], g fp32 [T][HV], beta bf16 [T][HV], A bf16 [T][HV][64] (row r written up to the end of its 16-column
 * block; other entries untouched). k . k^T runs on the bf16 matrix cores (exact products, fp32 accumulation); the
 * decay, mask, beta and the forward substitution run in fp32 (the reference uses bf16 / tf32 tensor-core products
 * and an approximate ex2: agreement with it is to that accuracy). Returns -1 for HV != 2H (the reference's code),
 * hipErrorInvalidConfiguration for NT or H <= 0 (an empty grid), hipErrorInvalidValue for missing or misaligned
 * buffers, else hipGetLastError(). */
int reax_kkt(const void* k, const void* g, const void* beta, void* A, const void* cu, const void* cidx, int NT, int H,
             int HV, void* stream);
/* Bytes of LDS the reax_kkt kernel uses (the reference returns its shared-memory size, reax_kkt.cu:272). */
int reax_kkt_smem(void);

/* Gated-DeltaNet chunked forward (skip form: blocks of A above the diagonal 16 x 16 blocks read as 0). Replaces
 * reax_howu, libreax_howu/reax_howu.cu:373-376. Per sequence (cu: int64 starts, N sequences) and value head hv (key
 * head hv / (HV/H)): the gated delta rule over 64-token chunks with the reference's bf16 rounding points. q, k bf16
 * [T][H][128]; v bf16 [T][HV][128]; beta bf16 [T][HV]; A bf16 [T][HV][64] (reax_kkt's output); g fp32 [T][HV] (the
 * chunk-local cumulative log2 decay); o bf16 [T][HV][128]. The products accumulate in fp32 on the matrix cores:
 * results agree with the reference's to bf16 accuracy. Returns hipErrorInvalidConfiguration for N or HV <= 0 (an
 * empty grid), hipErrorInvalidValue when H does not divide HV or a buffer is missing / misaligned, else
 * hipGetLastError(). */
int reax_howu(const void* q, const void* k, const void* v, const void* beta, const void* A, const void* g, void* o,
              const void* cu, float scale, int N, int H, int HV, void* stream);
/* The same (reax_howu.cu:367-370). */
int howu3_skip(const void* q, const void* k, const void* v, const void* beta, const void* A, const void* g, void* o,
               const void* cu, float scale, int N, int H, int HV, void* stream);
/* The dense form: every block of A is read (reax_howu.cu:363-366). */
int howu3_dense(const void* q, const void* k, const void* v, const void* beta, const void* A, const void* g, void* o,
                const void* cu, float scale, int N, int H, int HV, void* stream);
/* Bytes of LDS the chunked-forward kernel uses (the reference returns its shared-memory size, reax_howu.cu:371). */
int howu3_smem(void);
/* The chunked forward with the fused gated-RMSNorm epilogue. Replaces reax_howu_norm,
 * libreax_howu/reax_howu_norm_v3.cu:431-435: o is not stored; token t with R = f2s[t] >= 0 writes
 * out[R][hv][c] = bf16(bf16(nw[c] bf16(o[c] rr)) silu(z[R * ZS + hv * 128 + c])), rr = 1/sqrt(sum(o^2) factor + eps)
 * over the head's 128 values in the reference's order. rr and the SiLU exp are evaluated to fp32 accuracy where the
 * reference uses rsqrtf and expf. Return codes as reax_howu; also hipErrorInvalidValue for a missing or misaligned
 * f2s, z (8 bytes, ZS a multiple of 4) or nw. */
int reax_howu_norm(const void* q, const void* k, const void* v, const void* beta, const void* A, const void* g,
                   void* out, const void* cu, float scale, int N, int H, int HV, void* stream, const void* f2s,
                   const void* z, long long ZS, const void* nw, float eps, float factor);

#ifdef __cplusplus
}
#endif

#endif
