// fp32 / bf16 flash-attention backward on MFMA (gfx950).  Not yet enabled: the C-ABI
// routes every backward to the generic kernels while mfma_bwd_supported() is false.
#include "attn_launch.h"

namespace ctattn {

bool mfma_bwd_supported(int, int64_t) { return false; }

int64_t mfma_bwd_workspace_bytes(int, const AttnShape &) { return 0; }

hipError_t launch_mfma_bwd(int, const void *, const void *, const void *, const void *,
                           const float *, const float *, void *, void *, void *, void *,
                           const AttnShape &, hipStream_t) {
    return hipErrorNotSupported;
}

}  // namespace ctattn
