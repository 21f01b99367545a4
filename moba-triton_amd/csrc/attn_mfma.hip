// bf16 / fp16 MFMA kernels of the KV-block-major attention (gfx950).
#include "attn_common.h"

namespace moba {

int attend_mfma(const AttnArgs& a, int dtype, int acc_dtype, int64_t n_cols, hipStream_t st) {
  (void)a; (void)dtype; (void)acc_dtype; (void)n_cols; (void)st;
  return MOBA_ERR_UNSUPPORTED;
}

int bwd_mfma(const AttnArgs& a, int dtype, int acc_dtype, int64_t n_cols, hipStream_t st) {
  (void)a; (void)dtype; (void)acc_dtype; (void)n_cols; (void)st;
  return MOBA_ERR_UNSUPPORTED;
}

}  // namespace moba
