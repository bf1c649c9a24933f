/* C ABI of libreax_plain.so, the MI355X (gfx950) rebuild of the reference's plain GEMM library
 * (libreax_plain/gemm_plain2.cu). Caller-owned device pointers, asynchronous on `stream` (hipStream_t, NULL = default
 * stream). */
#ifndef LIBREAX_PLAIN_H
#define LIBREAX_PLAIN_H

#ifdef __cplusplus
extern "C" {
#endif

/* Number of config indices reax_gemm accepts (15, as gemm_plain2.cu:31). */
int reax_gemm_ncfg(void);
/* Name of config c, "?" outside 0..14 (gemm_plain2.cu:32-36). The index selects a CUTLASS tile shape in the
 * reference (all with the same results); here it selects one of the gfx950 matrix-core tiles (index 0: 256 x 256;
 * the others the tile nearest the reference config's shape), which the name describes. All give identical bits. */
const char* reax_gemm_cfgname(int c);
/* D[M][N] (row stride ldd) = bf16(X[M][K] W[N][K]^T) with fp32 accumulation; replaces reax_gemm, gemm_plain2.cu:37-56.
 * Returns 0 on success, 9 for an unknown cfg (as the reference), 1 for shapes the reference's kernels cannot take
 * (a size <= 0, K or ldd not a multiple of 8, ldd < N), a missing buffer or X / W not 16-byte aligned, 4 for a
 * launch error. K is summed in ascending 16-element MFMA steps: results agree with the reference's to fp32
 * accumulation accuracy, not bit for bit. */
int reax_gemm(int cfg, const void* x, const void* w, void* d, int M, int N, int K, int ldd, void* stream);

#ifdef __cplusplus
}
#endif
#endif
