// Mamba-2 SSD MFMA path (placeholder until the gfx950 kernel lands).
#include "ssd2.h"

namespace mamba {
bool ssd2_mfma_supported(const Ssd2Params&) { return false; }
size_t ssd2_mfma_workspace(const Ssd2Params&) { return 0; }
int ssd2_mfma_launch(const Ssd2Params&, void*, hipStream_t, hipEvent_t, hipEvent_t) {
    return MAMBA_ERR_UNSUPPORTED;
}
}  // namespace mamba
