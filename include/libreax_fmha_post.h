/* C ABI of libreax_fmha_post.so, the MI355X (gfx950) rebuild of the reference's fmha_post library.
 *
 * Exactly the three entry points of libreax_fmha_post/reax_fmha_v11.cu (v11:565-590), same names, argument
 * order, types, tensor layouts, error codes and stream semantics:
 *   - every pointer is caller-owned device memory; the library allocates nothing and keeps no pointer;
 *   - every stride is in elements; head_dim is fixed at 256 and its stride is 1 (v11:25);
 *   - H is the KV-head count and G the query heads per KV head: folded row r = m*G + g is query head h*G + g
 *     at token m (v11:452); qpos/inv are indexed by r / G;
 *   - the launch is asynchronous on `stream` (a hipStream_t; NULL = default stream); no host synchronisation;
 *   - returns 0, or the hipError_t code of the launch (the reference returns cudaGetLastError(), v11:563),
 *     or -1 when reax_fmha_b gets a NULL bias (v11:570). Arguments the kernels cannot address (row starts
 *     not 16-byte aligned, the reference's own precondition v11:227, 241, 249) return hipErrorInvalidValue.
 */
#ifndef LIBREAX_FMHA_POST_H
#define LIBREAX_FMHA_POST_H

#ifdef __cplusplus
extern "C" {
#endif

/* Additive-bias attention: O = softmax(scale * Q K^T + bias) V, every key visible.
 * Replaces reax_fmha_b, libreax_fmha_post/reax_fmha_v11.cu:565-573. */
int reax_fmha_b(const void* q, const void* k, const void* v, const void* bias, void* o, float scale, int B, int H,
                int M, int N, long long qsB, long long qsH, long long qsM, long long ksB, long long ksH, long long ksM,
                long long vsB, long long vsH, long long vsM, long long bsB, long long bsH, long long bsM,
                long long osB, long long osH, long long osM, void* stream);

/* qpos / causal GQA attention: row r of batch b sees keys 0..qpos[b*qpBs + r/G].
 * Replaces reax_fmha_q, libreax_fmha_post/reax_fmha_v11.cu:574-581. */
int reax_fmha_q(const void* q, const void* k, const void* v, const int* qpos, int G, long long qpBs, void* o,
                float scale, int B, int H, int M, int N, long long qsB, long long qsH, long long qsM, long long ksB,
                long long ksH, long long ksM, long long vsB, long long vsH, long long vsM, long long osB, long long osH,
                long long osM, void* stream);

/* qpos attention with the fused attn_post epilogue:
 *   out[inv[b*Lq + r/G]][(h*G + r%G)*256 + d] = bf16(bf16(o) * bf16(sigmoid(qg[R][h*G + r%G][256 + d])))
 * qg is [T][Hq][2*256] (the gate is the second half), out is [T][Hq*256]; rows with inv < 0 are not written.
 * Replaces reax_fmha_qp, libreax_fmha_post/reax_fmha_v11.cu:583-590. */
int reax_fmha_qp(const void* q, const void* k, const void* v, const int* qpos, int G, long long qpBs, float scale,
                 int B, int H, int M, int N, long long qsB, long long qsH, long long qsM, long long ksB, long long ksH,
                 long long ksM, long long vsB, long long vsH, long long vsM, const int* inv, int Lq, const void* qg,
                 long long qg_rs, void* outp, long long out_rs, void* stream);

#ifdef __cplusplus
}
#endif

#endif
