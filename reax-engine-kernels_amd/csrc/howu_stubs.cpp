// Gated-DeltaNet / norm / conv entry points of libreax_howu.so that are not implemented yet. They keep the
// reference prototypes (libreax_howu/reax_howu.cu:363-376, reax_howu_norm_v3.cu:431-435) so that a loader which
// resolves every symbol of the library still loads it, but launch nothing and return REAX_ERR_NOT_IMPLEMENTED.
// (reax_rarn is implemented in gdn_rarn.hip, reax_conv_l2 / reax_conv_v in gdn_conv.hip, reax_kkt in gdn_kkt.hip.)
#pragma GCC visibility push(default)
#include "libreax_howu.h"
#pragma GCC visibility pop

extern "C" {

int howu3_dense(const void*, const void*, const void*, const void*, const void*, const void*, void*, const void*,
                float, int, int, int, void*) {
  return REAX_ERR_NOT_IMPLEMENTED;
}
int howu3_skip(const void*, const void*, const void*, const void*, const void*, const void*, void*, const void*, float,
               int, int, int, void*) {
  return REAX_ERR_NOT_IMPLEMENTED;
}
int howu3_smem(void) { return 0; }
int reax_howu(const void*, const void*, const void*, const void*, const void*, const void*, void*, const void*, float,
              int, int, int, void*) {
  return REAX_ERR_NOT_IMPLEMENTED;
}
int reax_howu_norm(const void*, const void*, const void*, const void*, const void*, const void*, void*, const void*,
                   float, int, int, int, void*, const void*, const void*, long long, const void*, float, float) {
  return REAX_ERR_NOT_IMPLEMENTED;
}
}  // extern "C"
