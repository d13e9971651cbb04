// Attention forward and backward: the entry points, their contract checks, and the generic
// kernels (any dtype, any head width up to 256, f32 arithmetic, one wavefront per row). The
// MFMA kernels for bf16/f16 with D in {64, 128} live in attention_fwd.hip and
// attention_mfma_bwd.hip and are chosen here when they take the call.
#include <algorithm>
#include <string>

#include "attention_kernels.h"
#include "dm_common.h"

namespace dm {

// ------------------------------------------------------------------------------------------
// Generic forward: wave w of the block takes row (b, i, h); lanes split the head dimension.
// Online softmax in f32 over the keys of the row's interval (crates/dash-ops/src/attention/
// kernels.rs:683-997 computes the same with tiles; the reference, reference.rs:305-348, with
// the scores materialised).
// ------------------------------------------------------------------------------------------

template <int DT, int NPL>
__global__ __launch_bounds__(256) void attn_fwd_generic(MaskInfo m, int64_t B, int64_t Hq,
                                                        int64_t Hkv, int64_t D, float scale,
                                                        AttnStrides sd, const void *q,
                                                        const void *k, const void *v, void *o,
                                                        float *lse) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t Tq = m.tq, Tk = m.tk;
    if (row >= B * Tq * Hq) return;
    const int64_t h = row % Hq, i = (row / Hq) % Tq, b = row / (Hq * Tq);
    const int64_t kh = h / (Hq / Hkv);
    const int64_t qo = b * sd.q.b + i * sd.q.t + h * sd.q.h;
    float qr[NPL], acc[NPL];
#pragma unroll
    for (int e = 0; e < NPL; e++) {
        int64_t d = lane + 64 * e;
        qr[e] = d < D ? ld<DT>(q, qo + d) : 0.f;
        acc[e] = 0.f;
    }
    int64_t lo, hi;
    row_bounds(m, i, &lo, &hi);
    float mx = -INFINITY, l = 0.f;
    for (int64_t j = lo; j < hi; j++) {
        if (m.pad && m.pad[b * Tk + j]) continue;
        const int64_t kr = b * sd.k.b + j * sd.k.t + kh * sd.k.h;
        const int64_t vr = b * sd.v.b + j * sd.v.t + kh * sd.v.h;
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < NPL; e++) {
            int64_t d = lane + 64 * e;
            if (d < D) s += qr[e] * ld<DT>(k, kr + d);
        }
        s = wave_sum(s) * scale;
        float mn = fmaxf(mx, s);
        float alpha = expf(mx - mn), p = expf(s - mn);
        l = l * alpha + p;
#pragma unroll
        for (int e = 0; e < NPL; e++) {
            int64_t d = lane + 64 * e;
            float vv = d < D ? ld<DT>(v, vr + d) : 0.f;
            acc[e] = acc[e] * alpha + p * vv;
        }
        mx = mn;
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
    for (int e = 0; e < NPL; e++) {
        int64_t d = lane + 64 * e;
        if (d < D) st<DT>(o, row * D + d, acc[e] * inv);
    }
    if (lane == 0) lse[row] = l > 0.f ? mx + logf(l) : -INFINITY;
}

// ------------------------------------------------------------------------------------------
// Generic backward (reference.rs:352-431): delta = rowsum(dO * O); per query row
// dQ = scale sum_j P (dP - delta) K_j; per key row and key-value head dK = scale sum dS Q,
// dV = sum P dO over the group's query heads and the queries that see the key. Every output
// element is one wavefront's sequential sum: deterministic.
// ------------------------------------------------------------------------------------------

template <int DT, int NPL>
__global__ __launch_bounds__(256) void attn_delta_generic(int64_t rows, int64_t Tq, int64_t Hq,
                                                          int64_t D, AttnStrides sd,
                                                          const void *o, const void *d_o,
                                                          float *delta) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int64_t h = row % Hq, i = (row / Hq) % Tq, b = row / (Hq * Tq);
    const int64_t oo = b * sd.o.b + i * sd.o.t + h * sd.o.h;
    const int64_t go = b * sd.g.b + i * sd.g.t + h * sd.g.h;
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < NPL; e++) {
        int64_t d = lane + 64 * e;
        if (d < D) s += ld<DT>(o, oo + d) * ld<DT>(d_o, go + d);
    }
    s = wave_sum(s);
    if (lane == 0) delta[row] = s;
}

template <int DT, int NPL>
__global__ __launch_bounds__(256) void attn_dq_generic(MaskInfo m, int64_t B, int64_t Hq,
                                                       int64_t Hkv, int64_t D, float scale,
                                                       AttnStrides sd, const void *q,
                                                       const void *k, const void *v,
                                                       const float *lse, const void *d_o,
                                                       const float *delta, void *dq) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t Tq = m.tq, Tk = m.tk;
    if (row >= B * Tq * Hq) return;
    const int64_t h = row % Hq, i = (row / Hq) % Tq, b = row / (Hq * Tq);
    const int64_t kh = h / (Hq / Hkv);
    const int64_t qo = b * sd.q.b + i * sd.q.t + h * sd.q.h;
    const int64_t go = b * sd.g.b + i * sd.g.t + h * sd.g.h;
    float qr[NPL], gr[NPL], acc[NPL];
#pragma unroll
    for (int e = 0; e < NPL; e++) {
        int64_t d = lane + 64 * e;
        qr[e] = d < D ? ld<DT>(q, qo + d) : 0.f;
        gr[e] = d < D ? ld<DT>(d_o, go + d) : 0.f;
        acc[e] = 0.f;
    }
    const float ls = lse[row], dl = delta[row];
    int64_t lo, hi;
    row_bounds(m, i, &lo, &hi);
    if (ls == -INFINITY) hi = lo;  // a query that sees no key: dq = 0
    for (int64_t j = lo; j < hi; j++) {
        if (m.pad && m.pad[b * Tk + j]) continue;
        const int64_t kr = b * sd.k.b + j * sd.k.t + kh * sd.k.h;
        const int64_t vr = b * sd.v.b + j * sd.v.t + kh * sd.v.h;
        float s = 0.f, dp = 0.f;
#pragma unroll
        for (int e = 0; e < NPL; e++) {
            int64_t d = lane + 64 * e;
            if (d < D) {
                s += qr[e] * ld<DT>(k, kr + d);
                dp += gr[e] * ld<DT>(v, vr + d);
            }
        }
        s = wave_sum(s);
        dp = wave_sum(dp);
        const float p = expf(s * scale - ls);
        const float ds = p * (dp - dl);
#pragma unroll
        for (int e = 0; e < NPL; e++) {
            int64_t d = lane + 64 * e;
            if (d < D) acc[e] += ds * ld<DT>(k, kr + d);
        }
    }
#pragma unroll
    for (int e = 0; e < NPL; e++) {
        int64_t d = lane + 64 * e;
        if (d < D) st<DT>(dq, row * D + d, acc[e] * scale);
    }
}

template <int DT, int NPL>
__global__ __launch_bounds__(256) void attn_dkdv_generic(MaskInfo m, int64_t B, int64_t Hq,
                                                         int64_t Hkv, int64_t D, float scale,
                                                         AttnStrides sd, const void *q,
                                                         const void *k, const void *v,
                                                         const float *lse, const void *d_o,
                                                         const float *delta, void *dk,
                                                         void *dv) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t Tq = m.tq, Tk = m.tk;
    if (row >= B * Tk * Hkv) return;
    const int64_t kh = row % Hkv, j = (row / Hkv) % Tk, b = row / (Hkv * Tk);
    const int64_t group = Hq / Hkv;
    const int64_t ko = b * sd.k.b + j * sd.k.t + kh * sd.k.h;
    const int64_t vo = b * sd.v.b + j * sd.v.t + kh * sd.v.h;
    float kr[NPL], vr[NPL], ak[NPL], av[NPL];
#pragma unroll
    for (int e = 0; e < NPL; e++) {
        int64_t d = lane + 64 * e;
        kr[e] = d < D ? ld<DT>(k, ko + d) : 0.f;
        vr[e] = d < D ? ld<DT>(v, vo + d) : 0.f;
        ak[e] = av[e] = 0.f;
    }
    const bool padded = m.pad && m.pad[b * Tk + j];
    for (int64_t i = 0; i < Tq && !padded; i++) {
        int64_t lo, hi;
        row_bounds(m, i, &lo, &hi);
        if (j < lo || j >= hi) continue;
        for (int64_t h = kh * group; h < (kh + 1) * group; h++) {
            const int64_t qr = (b * Tq + i) * Hq + h;
            const float ls = lse[qr];
            if (ls == -INFINITY) continue;
            const int64_t qo = b * sd.q.b + i * sd.q.t + h * sd.q.h;
            const int64_t go = b * sd.g.b + i * sd.g.t + h * sd.g.h;
            float s = 0.f, dp = 0.f;
#pragma unroll
            for (int e = 0; e < NPL; e++) {
                int64_t d = lane + 64 * e;
                if (d < D) {
                    s += kr[e] * ld<DT>(q, qo + d);
                    dp += vr[e] * ld<DT>(d_o, go + d);
                }
            }
            s = wave_sum(s);
            dp = wave_sum(dp);
            const float p = expf(s * scale - ls);
            const float ds = p * (dp - delta[qr]);
#pragma unroll
            for (int e = 0; e < NPL; e++) {
                int64_t d = lane + 64 * e;
                if (d < D) {
                    ak[e] += ds * ld<DT>(q, qo + d);
                    av[e] += p * ld<DT>(d_o, go + d);
                }
            }
        }
    }
#pragma unroll
    for (int e = 0; e < NPL; e++) {
        int64_t d = lane + 64 * e;
        if (d < D) {
            st<DT>(dk, row * D + d, ak[e] * scale);
            st<DT>(dv, row * D + d, av[e]);
        }
    }
}

// ------------------------------------------------------------------------------------------
// Contract checks (check_shapes, crates/dash-ops/src/attention.rs:551-590)
// ------------------------------------------------------------------------------------------

int check_attention(const dm_attention_desc *d, const char *op) {
    std::string o(op);
    if (!d) return refuse(o + ": null descriptor");
    if (d->b < 0 || d->tq < 0 || d->tk < 0 || d->hq < 0 || d->hkv < 0 || d->d < 0)
        return refuse(o + ": negative dimension");
    if (d->hkv <= 0 || d->hq % d->hkv != 0)
        return refuse(o + ": the query heads (" + std::to_string(d->hq) +
                      ") must be a multiple of the key-value heads (" + std::to_string(d->hkv) +
                      ")");
    if (d->dtype != DM_F32 && d->dtype != DM_BF16 && d->dtype != DM_F16)
        return refuse(o + ": dtype must be f32, bf16 or f16");
    if (d->mask_kind == DM_MASK_KEY_PADDING && !d->key_padding && d->b * d->tk > 0)
        return refuse(o + ": the key padding mask is missing");
    if (d->mask_kind == DM_MASK_PACKED) {
        if (d->b != 1) return refuse(o + ": packed sequences lie along the time, B = 1");
        if (d->nseq < 1 || !d->cu_seqlens_q || !d->cu_seqlens_k)
            return refuse(o + ": cu_seqlens_q and cu_seqlens_k are [S + 1], one S");
    }
    if (d->mask_kind < 0 || d->mask_kind > 2) return refuse(o + ": unknown mask kind");
    if (d->strided) {
        const AttnStrides s = attn_strides(d);
        if (!strides_ok(s.q) || !strides_ok(s.k) || !strides_ok(s.v) || !strides_ok(s.o) ||
            !strides_ok(s.g))
            return refuse(o + ": strides must not be negative");
    }
    if (d->d > 256)
        return refuse(o + ": head dimension " + std::to_string(d->d) +
                      " above 256 is not implemented");
    return DM_OK;
}

static int npl_of(int64_t d) { return d <= 64 ? 1 : (d <= 128 ? 2 : 4); }

#define DM_DISPATCH_DT_NPL(DTV, NPLV, ...)                                              \
    switch ((DTV) * 8 + (NPLV)) {                                                       \
        case DM_F32 * 8 + 1: { constexpr int DT = DM_F32, NPL = 1; __VA_ARGS__; break; } \
        case DM_F32 * 8 + 2: { constexpr int DT = DM_F32, NPL = 2; __VA_ARGS__; break; } \
        case DM_F32 * 8 + 4: { constexpr int DT = DM_F32, NPL = 4; __VA_ARGS__; break; } \
        case DM_BF16 * 8 + 1: { constexpr int DT = DM_BF16, NPL = 1; __VA_ARGS__; break; } \
        case DM_BF16 * 8 + 2: { constexpr int DT = DM_BF16, NPL = 2; __VA_ARGS__; break; } \
        case DM_BF16 * 8 + 4: { constexpr int DT = DM_BF16, NPL = 4; __VA_ARGS__; break; } \
        case DM_F16 * 8 + 1: { constexpr int DT = DM_F16, NPL = 1; __VA_ARGS__; break; } \
        case DM_F16 * 8 + 2: { constexpr int DT = DM_F16, NPL = 2; __VA_ARGS__; break; } \
        case DM_F16 * 8 + 4: { constexpr int DT = DM_F16, NPL = 4; __VA_ARGS__; break; } \
        default: break;                                                                 \
    }

int launch_attn_fwd_generic(const MaskInfo &m, const dm_attention_desc *d, float scale,
                            const void *q, const void *k, const void *v, void *o, float *lse,
                            hipStream_t st) {
    const int64_t rows = d->b * d->tq * d->hq;
    if (rows == 0) return DM_OK;
    dim3 grid((unsigned)((rows + 3) / 4)), block(256);
    DM_DISPATCH_DT_NPL(d->dtype, npl_of(d->d),
                       attn_fwd_generic<DT, NPL><<<grid, block, 0, st>>>(
                           m, d->b, d->hq, d->hkv, d->d, scale, attn_strides(d), q, k, v, o,
                           lse));
    probe_add(DM_PROBE_ATTN_FWD_GENERIC);
    DM_LAUNCH_CHECK("attention: forward launch");
    return DM_OK;
}

}  // namespace dm

using namespace dm;

extern "C" {

size_t dm_attention_fwd_workspace(const dm_attention_desc *desc) {
    (void)desc;
    return 0;
}

int dm_attention_fwd(const dm_attention_desc *desc, const void *q, const void *k, const void *v,
                     void *o, float *lse, void *workspace, size_t workspace_bytes,
                     void *stream) {
    (void)workspace;
    (void)workspace_bytes;
    int rc = check_attention(desc, "attention");
    if (rc) return rc;
    hipStream_t st = (hipStream_t)stream;
    const MaskInfo m = mask_info(desc);
    const float scale = scale_of(desc);
    const int64_t rows = desc->b * desc->tq * desc->hq;
    if (rows == 0) return DM_OK;
    if (desc->tk == 0 || desc->d == 0) {
        // no key at all: zeros and a log-sum-exp of -inf (reference.rs:312-325)
        fill_zero(o, rows * desc->d * dtype_bytes(desc->dtype), st);
        fill_f32(lse, -INFINITY, rows, st);
        DM_LAUNCH_CHECK("attention: fill");
        return DM_OK;
    }
    if (mfma_fwd_takes(desc, q, k, v))
        return launch_attn_fwd_mfma(m, desc, scale, q, k, v, o, lse, st);
    return launch_attn_fwd_generic(m, desc, scale, q, k, v, o, lse, st);
}

size_t dm_attention_bwd_workspace(const dm_attention_desc *desc) {
    if (!desc) return 0;
    const size_t rows = (size_t)(desc->b * desc->tq * desc->hq);
    size_t bytes = align_up(rows * sizeof(float));  // delta
    return bytes + mfma_bwd_workspace(desc);
}

int dm_attention_bwd(const dm_attention_desc *desc, const void *q, const void *k, const void *v,
                     const void *o, const float *lse, const void *d_o, void *dq, void *dk,
                     void *dv, void *workspace, size_t workspace_bytes, void *stream) {
    int rc = check_attention(desc, "attention_backward");
    if (rc) return rc;
    if (workspace_bytes < dm_attention_bwd_workspace(desc))
        return refuse("attention_backward: the workspace is smaller than "
                      "dm_attention_bwd_workspace");
    hipStream_t st = (hipStream_t)stream;
    const MaskInfo m = mask_info(desc);
    const float scale = scale_of(desc);
    const int64_t qrows = desc->b * desc->tq * desc->hq, krows = desc->b * desc->tk * desc->hkv;
    const size_t eb = dtype_bytes(desc->dtype);
    if (qrows == 0 && krows == 0) return DM_OK;
    if (qrows == 0 || krows == 0 || desc->d == 0) {
        fill_zero(dq, qrows * desc->d * eb, st);
        fill_zero(dk, krows * desc->d * eb, st);
        fill_zero(dv, krows * desc->d * eb, st);
        DM_LAUNCH_CHECK("attention_backward: fill");
        return DM_OK;
    }
    float *delta = (float *)workspace;
    char *rest = (char *)workspace + align_up(qrows * sizeof(float));
    if (mfma_bwd_takes(desc, q, k, v, o, d_o))
        return launch_attn_bwd_mfma(m, desc, scale, q, k, v, o, lse, d_o, dq, dk, dv, delta,
                                    rest, st);
    const int npl = npl_of(desc->d);
    const AttnStrides sd = attn_strides(desc);
    dim3 block(256);
    DM_DISPATCH_DT_NPL(desc->dtype, npl,
        attn_delta_generic<DT, NPL><<<dim3((unsigned)((qrows + 3) / 4)), block, 0, st>>>(
            qrows, desc->tq, desc->hq, desc->d, sd, o, d_o, delta);
        attn_dq_generic<DT, NPL><<<dim3((unsigned)((qrows + 3) / 4)), block, 0, st>>>(
            m, desc->b, desc->hq, desc->hkv, desc->d, scale, sd, q, k, v, lse, d_o, delta, dq);
        attn_dkdv_generic<DT, NPL><<<dim3((unsigned)((krows + 3) / 4)), block, 0, st>>>(
            m, desc->b, desc->hq, desc->hkv, desc->d, scale, sd, q, k, v, lse, d_o, delta, dk,
            dv));
    probe_add(DM_PROBE_ATTN_BWD_GENERIC, 3);
    DM_LAUNCH_CHECK("attention_backward: launch");
    return DM_OK;
}

}  // extern "C"
