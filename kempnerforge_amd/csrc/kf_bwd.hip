// bf16 MFMA backward attention for gfx950 (head_dim 64 or 128).
#include "kf_common.h"
#include "kf_internal.h"

namespace kf {

bool bwd_mfma_supported(const BwdArgs&) { return false; }
size_t bwd_mfma_workspace(int, int, int, int, int) { return 0; }
int bwd_mfma(const BwdArgs&, void*) {
  set_error("MFMA backward not available");
  return KF_ERR_UNSUPPORTED;
}

}  // namespace kf
