// Compressed-state backward (placeholder until the fused kernels land).
#include "ep_common.h"
#include "ep_internal.h"

namespace ep {

size_t backward_workspace(int64_t, int64_t, int64_t, int, int) { return 0; }

int launch_backward(const PackedDesc &, const ActDesc &, const ActDesc &, int64_t, const OutDesc &,
                    float *, float *, int64_t, void *, size_t, hipStream_t)
{
    return set_error(EP_DECLINE_SHAPE, "backward not built yet");
}

}  // namespace ep
