// attn_bwd.hip -- flash-attention backward (placeholder until the kernels land).
#include "common.h"
#include "kernels.h"

namespace gonn {

size_t bwd_workspace_bytes(int, int, int, int) { return 0; }

hipError_t launch_bwd(const BwdParams&, int, int, int, const float*, void*, hipStream_t) {
    return hipErrorNotSupported;
}

}  // namespace gonn
