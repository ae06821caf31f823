// Matrix-core SDPA backward (bf16, head size 64 / 128).
#include "sdpa_common.h"

namespace mfx {

bool bwd_mfma_supports(const SdpaBwdParams& p) { return false; }

int launch_bwd_mfma(const SdpaBwdParams& p, hipStream_t s) {
  return fail(MFX_E_UNSUPPORTED, "matrix-core backward not available");
}

}  // namespace mfx
