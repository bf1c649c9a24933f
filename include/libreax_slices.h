/* C ABI of libreax_slices.so, the MI355X (gfx950) rebuild of the reference's split-K partial GEMM library
 * (libreax_slices/gemm_slices_v2.cu). Caller-owned device pointers, asynchronous on `stream` (hipStream_t, NULL =
 * default stream). */
#ifndef LIBREAX_SLICES_H
#define LIBREAX_SLICES_H

#ifdef __cplusplus
extern "C" {
#endif

/* Number of config indices reax_slices accepts (16, as gemm_slices_v2.cu:56). */
int reax_slices_ncfg(void);
/* Name of config c, "?" outside 0..15 (gemm_slices_v2.cu:57-64); the index selects one of the gfx950
 * matrix-core tiles (index 0: 256 x 256; the others the tile nearest the reference config's shape), which the name
 * describes. All give identical bits. */
const char* reax_slices_cfgname(int c);
/* Split-K partials: for s = 0..S-1, P[s][M][N] = X[:, s*kps .. (s+1)*kps) W[:, s*kps .. (s+1)*kps)^T with X [M][K]
 * and W [N][K] row-major, fp32 accumulation, each partial rounded once to fp32 (part_fp32 != 0) or bf16, partial s at
 * p + s*M*N elements. Replaces reax_slices, gemm_slices_v2.cu:65-84. Return codes as reax_gemm (9: unknown cfg; 1:
 * sizes <= 0, kps or K not a multiple of 8, N not a multiple of 8, S * kps > K, S > 65535, a missing buffer or X / W
 * not 16-byte aligned; 4: launch error). */
int reax_slices(int cfg, int part_fp32, const void* x, const void* w, void* p, int M, int N, int kps, int S, int K,
                void* stream);

#ifdef __cplusplus
}
#endif
#endif
