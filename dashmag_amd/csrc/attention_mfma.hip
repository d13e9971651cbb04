// MFMA attention kernels (placeholder until the gfx950 kernels land: nothing is taken).
#include "attention_kernels.h"

namespace dm {

bool mfma_fwd_takes(const dm_attention_desc *d) { (void)d; return false; }
int launch_attn_fwd_mfma(const MaskInfo &, const dm_attention_desc *, float, const void *,
                         const void *, const void *, void *, float *, hipStream_t) {
    return refuse("attention: no MFMA kernel");
}
bool mfma_bwd_takes(const dm_attention_desc *d) { (void)d; return false; }
size_t mfma_bwd_workspace(const dm_attention_desc *d) { (void)d; return 0; }
int launch_attn_bwd_mfma(const MaskInfo &, const dm_attention_desc *, float, const void *,
                         const void *, const void *, const void *, const float *, const void *,
                         void *, void *, void *, float *, void *, hipStream_t) {
    return refuse("attention_backward: no MFMA kernel");
}

}  // namespace dm
