// Native scaled-MFMA MXFP4 path (v_mfma_scale_f32_*_f8f6f4).  Not built yet:
// the entry point reports LMOE_ERR_UNSUPPORTED so callers fall back to nothing
// silently -- the Python layer raises NotImplementedError.
#include "gemm_tile.h"

namespace lmoe {
namespace gemm {

int run_mxfp4_scaled(const Params& p, int epi, hipStream_t st, const char* name) {
  (void)p;
  (void)epi;
  (void)st;
  return fail(LMOE_ERR_UNSUPPORTED, "%s: scaled-MFMA mode is not implemented yet", name);
}

}  // namespace gemm
}  // namespace lmoe
