// Attention decode against a key-value cache (crates/dash-ops/src/attention.rs:732,
// attention/cube.rs:1126-1214, kernels.rs:2052-2239): flash-decoding. Pass 1 splits each
// sequence's keys into fixed-size spans; one workgroup reads a span of K and V rows once for
// all the query heads of a key-value head's group (the GQA reuse), and writes a normalised
// partial output and its log-sum-exp in f32. Pass 2 merges the spans by their log-sum-exp.
//
// Bandwidth-bound, no MFMA: each K/V row (D * 2 bytes) is read by D / 8 lanes with 16-byte
// loads, one wavefront covering 64 * 8 / D rows per load, the dot products reduced across the
// row's lanes with xor shuffles; f32 online softmax per lane group.
#include <string>

#include "attention_kernels.h"
#include "dm_common.h"

namespace dm {

constexpr int kDecodeSpan = 256;  // keys per workgroup (split)

struct Bf16x8 {
    uint4 raw;
};

template <int DT>
__device__ __forceinline__ void unpack8(const uint4 &r, float *x) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
        if (DT == DM_BF16) {
            x[2 * e] = __uint_as_float(w[e] << 16);
            x[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
        } else {
            union {
                uint32_t u;
                _Float16 h[2];
            } c;
            c.u = w[e];
            x[2 * e] = (float)c.h[0];
            x[2 * e + 1] = (float)c.h[1];
        }
    }
}

// One split of one (sequence, key-value head): keys [base + split * span, ...) of the keys the
// sequence's query sees, [lo, hi). Writes part_o [B, Hq, nsplit, D] (normalised) and part_lse
// [B, Hq, nsplit] (-inf for a split that sees nothing).
template <int DT, int D, int G>
__global__ __launch_bounds__(256) void decode_split(int64_t S, int64_t Hq, int64_t Hkv,
                                                    int64_t left, float scale, int nsplit,
                                                    const void *__restrict__ q,
                                                    const void *__restrict__ k,
                                                    const void *__restrict__ v,
                                                    const int32_t *__restrict__ lengths,
                                                    float *__restrict__ part_o,
                                                    float *__restrict__ part_lse) {
    constexpr int LPR = D / 8;       // lanes per K/V row
    constexpr int RPW = 64 / LPR;    // rows per wavefront per step
    constexpr int NW = 4;            // wavefronts
    constexpr int GROUPS = RPW * NW; // independent partial states in the workgroup
    const int split = blockIdx.x, kh = blockIdx.y;
    const int64_t b = blockIdx.z;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane / LPR, seg = lane % LPR;

    int64_t len = lengths ? (int64_t)lengths[b] : S;
    if (len > S) len = S;
    if (len < 0) len = 0;
    int64_t lo = left >= 0 ? len - 1 - left : 0;
    if (lo < 0) lo = 0;
    const int64_t start = lo + (int64_t)split * kDecodeSpan;
    int64_t end = start + kDecodeSpan;
    if (end > len) end = len;

    // queries of the group, this lane's 8 elements, pre-scaled by scale * log2(e)
    const float qscale = scale * 1.4426950408889634f;
    float qv[G][8];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const int64_t h = kh * G + g;
        const uint4 raw = *(const uint4 *)((const char *)q + ((b * Hq + h) * D + seg * 8) * 2);
        unpack8<DT>(raw, qv[g]);
#pragma unroll
        for (int e = 0; e < 8; e++) qv[g][e] *= qscale;
    }

    float mx[G], l[G], acc[G][8];
#pragma unroll
    for (int g = 0; g < G; g++) {
        mx[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) acc[g][e] = 0.f;
    }

    const int64_t row_stride = Hkv * D * 2;  // bytes between consecutive keys
    const char *kb = (const char *)k + (b * S * Hkv + kh) * D * 2 + seg * 16;
    const char *vb = (const char *)v + (b * S * Hkv + kh) * D * 2 + seg * 16;

    for (int64_t j0 = start + wave * RPW; j0 < end; j0 += NW * RPW * 2) {
        // two rows per lane group per step, loads issued before use
        const int64_t ja = j0 + r, jb = j0 + NW * RPW + r;
        const bool va = ja < end, vbv = jb < end;
        uint4 ka = make_uint4(0, 0, 0, 0), vra = ka, kbr = ka, vrb = ka;
        if (va) {
            ka = *(const uint4 *)(kb + ja * row_stride);
            vra = *(const uint4 *)(vb + ja * row_stride);
        }
        if (vbv) {
            kbr = *(const uint4 *)(kb + jb * row_stride);
            vrb = *(const uint4 *)(vb + jb * row_stride);
        }
        float kf[2][8], vf[2][8];
        unpack8<DT>(ka, kf[0]);
        unpack8<DT>(kbr, kf[1]);
        unpack8<DT>(vra, vf[0]);
        unpack8<DT>(vrb, vf[1]);
        float s[2][G];
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int g = 0; g < G; g++) {
                float t = 0.f;
#pragma unroll
                for (int e = 0; e < 8; e++) t += qv[g][e] * kf[u][e];
#pragma unroll
                for (int o = LPR / 2; o >= 1; o >>= 1) t += __shfl_xor(t, o, 64);
                s[u][g] = t;
            }
        if (!va) {
#pragma unroll
            for (int g = 0; g < G; g++) s[0][g] = -INFINITY;
        }
        if (!vbv) {
#pragma unroll
            for (int g = 0; g < G; g++) s[1][g] = -INFINITY;
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float mn = fmaxf(mx[g], fmaxf(s[0][g], s[1][g]));
            if (mn == -INFINITY) continue;
            const float alpha = exp2f(mx[g] - mn);
            const float p0 = exp2f(s[0][g] - mn), p1 = exp2f(s[1][g] - mn);
            l[g] = l[g] * alpha + p0 + p1;
#pragma unroll
            for (int e = 0; e < 8; e++) acc[g][e] = acc[g][e] * alpha + p0 * vf[0][e] + p1 * vf[1][e];
            mx[g] = mn;
        }
    }

    // Combine the GROUPS partial states through LDS: [GROUPS][G] (m, l), [GROUPS][G][D] acc.
    __shared__ float sm_m[GROUPS][G], sm_l[GROUPS][G];
    __shared__ float sm_acc[GROUPS][G][D];
    const int grp = wave * RPW + r;
#pragma unroll
    for (int g = 0; g < G; g++) {
        if (seg == 0) {
            sm_m[grp][g] = mx[g];
            sm_l[grp][g] = l[g];
        }
#pragma unroll
        for (int e = 0; e < 8; e++) sm_acc[grp][g][seg * 8 + e] = acc[g][e];
    }
    __syncthreads();
    for (int x = threadIdx.x; x < G * D; x += 256) {
        const int g = x / D, d = x % D;
        float M = -INFINITY;
        for (int t = 0; t < GROUPS; t++) M = fmaxf(M, sm_m[t][g]);
        float L = 0.f, A = 0.f;
        if (M != -INFINITY) {
            for (int t = 0; t < GROUPS; t++) {
                const float w = exp2f(sm_m[t][g] - M);
                L += sm_l[t][g] * w;
                A += sm_acc[t][g][d] * w;
            }
        }
        const int64_t h = kh * G + g;
        const int64_t pr = (b * Hq + h) * nsplit + split;
        part_o[pr * D + d] = L > 0.f ? A / L : 0.f;
        // natural-log lse of the split from the base-2 running maximum
        if (d == 0) part_lse[pr] = L > 0.f ? (M + log2f(L)) * 0.6931471805599453f : -INFINITY;
    }
}

// Pass 2: merges the splits of one (sequence, query head) by their log-sum-exp.
template <int DT>
__global__ __launch_bounds__(256) void decode_merge(int64_t rows, int64_t D, int nsplit,
                                                    const float *__restrict__ part_o,
                                                    const float *__restrict__ part_lse,
                                                    void *__restrict__ o) {
    const int64_t row = blockIdx.x;
    if (row >= rows) return;
    const float *pl = part_lse + row * nsplit;
    float M = -INFINITY;
    for (int s = 0; s < nsplit; s++) M = fmaxf(M, pl[s]);
    for (int64_t d = threadIdx.x; d < D; d += blockDim.x) {
        float L = 0.f, A = 0.f;
        if (M != -INFINITY) {
            for (int s = 0; s < nsplit; s++) {
                const float w = __expf(pl[s] - M);
                L += w;
                A += w * part_o[(row * nsplit + s) * D + d];
            }
        }
        st<DT>(o, row * D + d, L > 0.f ? A / L : 0.f);
    }
}

// The generic decode: the generic attention forward's arithmetic, one wavefront per
// (sequence, query head), for head widths and groups the split kernel does not take.
template <int DT, int NPL>
__global__ __launch_bounds__(256) void decode_generic(int64_t B, int64_t S, int64_t Hq,
                                                      int64_t Hkv, int64_t D, int64_t left,
                                                      float scale, const void *q, const void *k,
                                                      const void *v, const int32_t *lengths,
                                                      void *o) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= B * Hq) return;
    const int64_t b = row / Hq, h = row % Hq, kh = h / (Hq / Hkv);
    int64_t len = lengths ? (int64_t)lengths[b] : S;
    if (len > S) len = S;
    if (len < 0) len = 0;
    int64_t lo = left >= 0 ? len - 1 - left : 0;
    if (lo < 0) lo = 0;
    float qr[NPL], acc[NPL];
#pragma unroll
    for (int e = 0; e < NPL; e++) {
        int64_t d = lane + 64 * e;
        qr[e] = d < D ? ld<DT>(q, row * D + d) : 0.f;
        acc[e] = 0.f;
    }
    float mx = -INFINITY, l = 0.f;
    for (int64_t j = lo; j < len; j++) {
        const int64_t kr = ((b * S + j) * Hkv + kh) * D;
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < NPL; e++) {
            int64_t d = lane + 64 * e;
            if (d < D) s += qr[e] * ld<DT>(k, kr + d);
        }
        s = wave_sum(s) * scale;
        const float mn = fmaxf(mx, s);
        const float alpha = expf(mx - mn), p = expf(s - mn);
        l = l * alpha + p;
#pragma unroll
        for (int e = 0; e < NPL; e++) {
            int64_t d = lane + 64 * e;
            acc[e] = acc[e] * alpha + p * (d < D ? ld<DT>(v, kr + d) : 0.f);
        }
        mx = mn;
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
    for (int e = 0; e < NPL; e++) {
        int64_t d = lane + 64 * e;
        if (d < D) st<DT>(o, row * D + d, acc[e] * inv);
    }
}

static bool split_takes(const dm_attention_desc *d) {
    const int64_t g = d->hq / d->hkv;
    return (d->dtype == DM_BF16 || d->dtype == DM_F16) &&
           (d->d == 64 || d->d == 128 || d->d == 256) && (g == 1 || g == 2 || g == 4 || g == 8);
}

static int nsplit_of(const dm_attention_desc *d) {
    return (int)((d->tk + kDecodeSpan - 1) / kDecodeSpan);
}

static int64_t left_of(const dm_attention_desc *d) {
    const uint64_t span = (uint64_t)d->tk + 1;  // `bound(left, s + 1)`, reference.rs:449
    const uint64_t left = d->options.has_window ? d->options.window_left : DM_UNBOUNDED;
    return left < span ? (int64_t)left : -1;
}

}  // namespace dm

using namespace dm;

extern "C" {

size_t dm_attention_decode_workspace(const dm_attention_desc *d) {
    if (!d || !split_takes(d)) return 0;
    const size_t parts = (size_t)(d->b * d->hq) * nsplit_of(d);
    return align_up(parts * d->d * sizeof(float)) + align_up(parts * sizeof(float));
}

int dm_attention_decode(const dm_attention_desc *d, const void *q, const void *k, const void *v,
                        const int32_t *lengths, void *o, void *workspace, size_t workspace_bytes,
                        void *stream) {
    if (!d) return refuse("attention_decode: null descriptor");
    if (d->b < 0 || d->tk < 0 || d->hq < 0 || d->hkv <= 0 || d->d < 0)
        return refuse("attention_decode: bad dimensions");
    if (d->hq % d->hkv != 0)
        return refuse("attention_decode: the query heads (" + std::to_string(d->hq) +
                      ") must be a multiple of the key-value heads (" + std::to_string(d->hkv) +
                      ")");
    if (d->dtype != DM_F32 && d->dtype != DM_BF16 && d->dtype != DM_F16)
        return refuse("attention_decode: dtype must be f32, bf16 or f16");
    if (d->d > 256) return refuse("attention_decode: head dimension above 256 is not implemented");
    if (workspace_bytes < dm_attention_decode_workspace(d))
        return refuse("attention_decode: the workspace is smaller than dm_attention_decode_workspace");
    hipStream_t st = (hipStream_t)stream;
    const int64_t rows = d->b * d->hq;
    if (rows == 0 || d->d == 0) return DM_OK;
    const float scale = scale_of(d);
    const int64_t left = left_of(d);
    if (d->tk == 0) {
        fill_zero(o, rows * d->d * dtype_bytes(d->dtype), st);
        DM_LAUNCH_CHECK("attention_decode: fill");
        return DM_OK;
    }
    if (!split_takes(d)) {
        const int npl = d->d <= 64 ? 1 : (d->d <= 128 ? 2 : 4);
        dim3 grid((unsigned)((rows + 3) / 4));
#define DEC_GEN(DT, NPL)                                                                    \
    decode_generic<DT, NPL><<<grid, 256, 0, st>>>(d->b, d->tk, d->hq, d->hkv, d->d, left,   \
                                                  scale, q, k, v, lengths, o)
        if (d->dtype == DM_F32) {
            if (npl == 1) DEC_GEN(DM_F32, 1); else if (npl == 2) DEC_GEN(DM_F32, 2); else DEC_GEN(DM_F32, 4);
        } else if (d->dtype == DM_BF16) {
            if (npl == 1) DEC_GEN(DM_BF16, 1); else if (npl == 2) DEC_GEN(DM_BF16, 2); else DEC_GEN(DM_BF16, 4);
        } else {
            if (npl == 1) DEC_GEN(DM_F16, 1); else if (npl == 2) DEC_GEN(DM_F16, 2); else DEC_GEN(DM_F16, 4);
        }
#undef DEC_GEN
        probe_add(DM_PROBE_ATTN_FWD_GENERIC);
        DM_LAUNCH_CHECK("attention_decode: launch");
        return DM_OK;
    }
    const int nsplit = nsplit_of(d);
    const size_t parts = (size_t)rows * nsplit;
    float *part_o = (float *)workspace;
    float *part_lse = (float *)((char *)workspace + align_up(parts * d->d * sizeof(float)));
    dim3 grid(nsplit, (unsigned)d->hkv, (unsigned)d->b);
    const int g = (int)(d->hq / d->hkv);
#define DEC_SPLIT(DT, DD, GG)                                                               \
    decode_split<DT, DD, GG><<<grid, 256, 0, st>>>(d->tk, d->hq, d->hkv, left, scale, nsplit, \
                                                   q, k, v, lengths, part_o, part_lse)
#define DEC_G(DT, DD)                                \
    switch (g) {                                     \
        case 1: DEC_SPLIT(DT, DD, 1); break;         \
        case 2: DEC_SPLIT(DT, DD, 2); break;         \
        case 4: DEC_SPLIT(DT, DD, 4); break;         \
        default: DEC_SPLIT(DT, DD, 8); break;        \
    }
#define DEC_D(DT)                                    \
    switch (d->d) {                                  \
        case 64: DEC_G(DT, 64); break;               \
        case 128: DEC_G(DT, 128); break;             \
        default: DEC_G(DT, 256); break;              \
    }
    if (d->dtype == DM_BF16) {
        DEC_D(DM_BF16);
        decode_merge<DM_BF16><<<(unsigned)rows, 128, 0, st>>>(rows, d->d, nsplit, part_o, part_lse, o);
    } else {
        DEC_D(DM_F16);
        decode_merge<DM_F16><<<(unsigned)rows, 128, 0, st>>>(rows, d->d, nsplit, part_o, part_lse, o);
    }
#undef DEC_D
#undef DEC_G
#undef DEC_SPLIT
    probe_add(DM_PROBE_DECODE_SPLIT);
    probe_add(DM_PROBE_DECODE_MERGE);
    DM_LAUNCH_CHECK("attention_decode: launch");
    return DM_OK;
}

}  // extern "C"
