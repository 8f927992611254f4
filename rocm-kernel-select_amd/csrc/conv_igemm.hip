// MFMA implicit-GEMM conv kernels (placeholder table until the kernels land).
#include "conv_common.h"

namespace atk {

int conv_igemm_num_variants() { return 0; }
const char* conv_igemm_variant_name(int) { return nullptr; }
size_t conv_igemm_workspace_bytes(const ConvShape&, int) { return 0; }
int conv_igemm_launch(const ConvShape&, const void*, const void*, const void*, void*, int, void*,
                      size_t, hipStream_t) {
  return fail(ATK_UNSUPPORTED, "conv: no implicit-GEMM variants in this build");
}

}  // namespace atk
