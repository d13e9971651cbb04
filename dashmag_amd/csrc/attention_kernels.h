// Declarations shared by the attention translation units.
#pragma once

#include "dm_common.h"

namespace dm {

inline size_t dtype_bytes(int dt) { return dt == DM_F32 ? 4 : 2; }

// Fill kernels (graph-capture safe: no memset nodes).
void fill_f32(float *p, float value, int64_t n, hipStream_t st);
void fill_zero(void *p, size_t bytes, hipStream_t st);

int check_attention(const dm_attention_desc *d, const char *op);
int launch_attn_fwd_generic(const MaskInfo &m, const dm_attention_desc *d, float scale,
                            const void *q, const void *k, const void *v, void *o, float *lse,
                            hipStream_t st);

// MFMA paths (attention_fwd.hip, attention_mfma_bwd.hip): bf16/f16, D in {64, 128}.
bool rows_fit_32bit(const Strd &x, int64_t rows, int64_t d);
bool mfma_fwd_takes(const dm_attention_desc *d, const void *q, const void *k, const void *v);
int launch_attn_fwd_mfma(const MaskInfo &m, const dm_attention_desc *d, float scale,
                         const void *q, const void *k, const void *v, void *o, float *lse,
                         hipStream_t st);
bool mfma_bwd_takes(const dm_attention_desc *d, const void *q, const void *k, const void *v,
                    const void *o, const void *d_o);
size_t mfma_bwd_workspace(const dm_attention_desc *d);
int launch_attn_bwd_mfma(const MaskInfo &m, const dm_attention_desc *d, float scale,
                         const void *q, const void *k, const void *v, const void *o,
                         const float *lse, const void *d_o, void *dq, void *dk, void *dv,
                         float *delta, void *workspace, hipStream_t st);

}  // namespace dm
