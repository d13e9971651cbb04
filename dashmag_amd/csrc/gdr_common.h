// Declarations shared by the gated-delta-rule translation units.
#pragma once

#include "dm_common.h"

namespace dm {

constexpr int kChunk = 64;  // tokens per chunk (chunk/reference.rs:26)

struct GdrArgs {
    int64_t H, Dk, Dv;
    int64_t rows;  // B * T token rows of the inputs
    int g_dt, beta_dt, l2norm;
    float scale;
    const void *q, *k, *v, *g, *beta;
};

// The generic kernels' workspace: the plan, then per (chunk, head) f32 intermediates.
struct GdrWs {
    int32_t *seq_chunk0, *chunk_seq, *chunk_tok0, *chunk_len;
    float *G, *qn, *kn, *W, *U, *Sc, *Vn;
    float *Tm, *Am, *dvl, *dSn, *dVn, *ds, *gq, *gk, *gx;
};

int check_gdr(const dm_gdr_desc *d, const char *op, bool step);
// The chunk plan over the call's sequences (gdr_chunk.hip).
int launch_plan(const dm_gdr_desc *d, int32_t *seq_chunk0, int32_t *chunk_seq,
                int32_t *chunk_tok0, int32_t *chunk_len, hipStream_t st);
int64_t gdr_nseq(const dm_gdr_desc *d);
int64_t gdr_chunk_bound(const dm_gdr_desc *d);

// MFMA forward (gdr_chunk_mfma.hip): bf16/f16, Dk = Dv = 128.
bool gdr_mfma_takes(const dm_gdr_desc *d);
size_t gdr_mfma_fwd_workspace(const dm_gdr_desc *d);
int launch_gdr_mfma_fwd(const dm_gdr_desc *d, const void *q, const void *k, const void *v,
                        const void *g, const void *beta, const float *h0, void *out,
                        float *final_state, void *workspace, hipStream_t st);
size_t gdr_mfma_bwd_workspace(const dm_gdr_desc *d);
int launch_gdr_mfma_bwd(const dm_gdr_desc *d, const void *q, const void *k, const void *v,
                        const void *g, const void *beta, const float *h0, const void *d_out,
                        const float *d_final, void *dq, void *dk, void *dv, void *dg,
                        void *dbeta, float *dh0, void *workspace, hipStream_t st);
GdrArgs gdr_args(const dm_gdr_desc *d, const void *q, const void *k, const void *v,
                 const void *g, const void *beta);

}  // namespace dm
