// MFMA chunked gated delta rule forward (placeholder until the gfx950 kernels land).
#include "gdr_common.h"

namespace dm {

bool gdr_mfma_takes(const dm_gdr_desc *d) { (void)d; return false; }
size_t gdr_mfma_fwd_workspace(const dm_gdr_desc *d) { (void)d; return 0; }
int launch_gdr_mfma_fwd(const dm_gdr_desc *, const void *, const void *, const void *,
                        const void *, const void *, const float *, void *, float *, void *,
                        hipStream_t) {
    return refuse("chunk_gated_delta_rule: no MFMA kernel");
}

}  // namespace dm
