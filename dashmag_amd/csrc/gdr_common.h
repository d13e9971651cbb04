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
    // element strides of the inputs along their token rows (the flattened b * T + t) and heads:
    // q, k, v, g, beta and the backward's output gradient (o)
    int64_t q_t, q_h, k_t, k_h, v_t, v_h, g_t, g_h, b_t, b_h, o_t, o_h;
};

// Element offsets of token row `tok`, head h of each input.
__host__ __device__ inline int64_t q_at(const GdrArgs &a, int64_t tok, int64_t h) {
    return tok * a.q_t + h * a.q_h;
}
__host__ __device__ inline int64_t k_at(const GdrArgs &a, int64_t tok, int64_t h) {
    return tok * a.k_t + h * a.k_h;
}
__host__ __device__ inline int64_t v_at(const GdrArgs &a, int64_t tok, int64_t h) {
    return tok * a.v_t + h * a.v_h;
}
__host__ __device__ inline int64_t g_at(const GdrArgs &a, int64_t tok, int64_t h) {
    return tok * a.g_t + h * a.g_h;
}
__host__ __device__ inline int64_t b_at(const GdrArgs &a, int64_t tok, int64_t h) {
    return tok * a.b_t + h * a.b_h;
}
__host__ __device__ inline int64_t o_at(const GdrArgs &a, int64_t tok, int64_t h) {
    return tok * a.o_t + h * a.o_h;
}
// Whether the descriptor's strides index tokens as rows b * T + t (b stride = T x t stride, or
// a batch of one), each stride non-negative; `fast16` also asks 16-byte rows (multiples of 8
// elements for the vectors, the MFMA kernels' loads).
bool gdr_strides_ok(const dm_gdr_desc *d, bool step);
bool gdr_strides_16b(const dm_gdr_desc *d);

// The generic kernels' workspace: the plan, then per (chunk, head) f32 intermediates.
struct GdrWs {
    int32_t *seq_chunk0, *chunk_seq, *chunk_tok0, *chunk_len;
    float *G, *qn, *kn, *W, *U, *Sc, *Vn;
    float *Tm, *Am, *dvl, *dSn, *dVn, *ds, *gq, *gk, *gx;
};

int check_gdr(const dm_gdr_desc *d, const char *op, bool step);
// The chunk plan over the call's sequences (gdr_chunk.hip).
// seq_order (optional, [nseq]): the sequences by chunk count, the most first (ties by index),
// for at most kOrderMax sequences; the identity beyond.
constexpr int64_t kOrderMax = 4096;
int launch_plan(const dm_gdr_desc *d, int32_t *seq_chunk0, int32_t *chunk_seq,
                int32_t *chunk_tok0, int32_t *chunk_len, hipStream_t st,
                int32_t *seq_order = nullptr);
int64_t gdr_nseq(const dm_gdr_desc *d);
int64_t gdr_chunk_bound(const dm_gdr_desc *d);

// MFMA forward and backward (gdr_chunk_mfma.hip): bf16/f16, Dk and Dv multiples of 8 up to 128
// (the products are 128 wide; columns past a width are held at zero).
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
                 const void *g, const void *beta, bool step = false);

}  // namespace dm
