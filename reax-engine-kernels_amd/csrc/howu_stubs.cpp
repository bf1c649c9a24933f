// The Gated-DeltaNet entry point of libreax_howu.so that is not implemented yet, reax_howu_norm. It keeps the reference
// prototype (libreax_howu/reax_howu_norm_v3.cu:431-435) so that a loader which resolves every symbol of the library
// still loads it, but launches nothing and returns REAX_ERR_NOT_IMPLEMENTED. (reax_rarn is implemented in
// gdn_rarn.hip, reax_conv_l2 / reax_conv_v in gdn_conv.hip, reax_kkt in gdn_kkt.hip, reax_howu / howu3_* in
// gdn_howu.hip.)
#pragma GCC visibility push(default)
#include "libreax_howu.h"
#pragma GCC visibility pop

extern "C" {

int reax_howu_norm(const void*, const void*, const void*, const void*, const void*, const void*, void*, const void*,
                   float, int, int, int, void*, const void*, const void*, long long, const void*, float, float) {
  return REAX_ERR_NOT_IMPLEMENTED;
}
}  // extern "C"
