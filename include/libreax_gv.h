/* C ABI of libreax_gv.so, the MI355X (gfx950) rebuild of the reference's gate/up GEMM library
 * (libreax_gv/gateup_vis2.cu). Caller-owned device pointers, asynchronous on `stream` (hipStream_t, NULL = default
 * stream); the library allocates nothing. */
#ifndef LIBREAX_GV_H
#define LIBREAX_GV_H

#ifdef __cplusplus
extern "C" {
#endif

/* Number of config indices reax_gv accepts (20, as gateup_vis2.cu:172). */
int reax_gv_ncfg(void);
/* Name of config c, "?" outside 0..19 (gateup_vis2.cu:173-181); the index selects one of the
 * gfx950 matrix-core tiles (index 0: 256 x 256; the others the tile nearest the reference config's shape), which the
 * name describes. All give identical bits. */
const char* reax_gv_cfgname(int c);
/* out[M][N2] = bf16(bf16(silu(bf16(g))) * bf16(u)) with [g | u] = X[M][K] W[2*N2][K]^T, W's rows interleaving 4 gate
 * and 4 up rows per group of 4 output features (gateup_vis2.cu:1-6); replaces reax_gv, gateup_vis2.cu:182-208.
 * Returns 0 on success, 9 for an unknown cfg, 1 for K not a multiple of 8 or N2 not a multiple of 4 (as the
 * reference), 3 for sizes <= 0, missing or misaligned buffers (rows 16-byte aligned) or a launch error. fp32
 * accumulation in the matrix cores' order: agreement with the reference's to fp32 accumulation accuracy. */
int reax_gv(int cfg, const void* x, const void* w, void* out, int M, int N2, int K, void* stream);

#ifdef __cplusplus
}
#endif
#endif
