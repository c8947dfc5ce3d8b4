// expert_mfma_kernels.hip -- grouped expert GEMMs for large token counts
// (prefill) on int8 MFMA.  Placeholder launcher until the tiled kernel lands.
#include "qmoe_device.h"
#include "qmoe_internal.h"

namespace qmoe {

hipError_t launch_experts_mfma(const LayerDesc&, const Workspace&, int, hipStream_t) {
    return hipErrorNotSupported;
}

}  // namespace qmoe
