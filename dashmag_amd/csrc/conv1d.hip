// The causal depthwise conv1d (crates/dash-contract/src/conv1d.rs; dash-ops' CausalConv1dBackend,
// crates/dash-ops/src/conv1d.rs:198-360, kernels in conv1d/cube.rs) on gfx950: forward,
// backward and the decoding step, bandwidth-bound elementwise work without MFMA.
//
// Per sequence and channel c, with h the history (the initial state's W steps, then the inputs,
// zeros before those) and K the kernel width:
//   y[t, c] = sum_{j < K} weight[c, j] h[t - (K - 1) + j, c] (+ bias[c]);  out = y or SiLU(y).
//
// Layout: x, out, gradients [B, T, C] (C fastest), weight [C, K], bias [C], states [S, W, C] f32.
// A thread owns one 16-byte vector of channels (8 of a 16-bit dtype, 4 of f32; one channel when
// C is not a multiple of that) over a segment of consecutive steps, holding the taps and a
// sliding window of the last K - 1 inputs in registers, so x is read from HBM once (plus K - 1
// steps per segment) and the output written once; consecutive threads read consecutive 16-byte
// pieces of a row. Segments may cross sequence boundaries (packed sequences): the window is
// refilled from the initial state, or zeros, at each sequence's first step.
//
// The backward sweeps each sequence's part of a segment from its last step to its first, with a
// window of the next K - 1 steps' pre-activation gradients: the input gradient of step t is
// sum_j weight[j] dy[t + K - 1 - j]. The weight and bias gradients are summed per thread over
// its segment, written as per-segment partials, and summed over the segments in a fixed order by
// a second kernel (deterministic). Kernel widths 1..8 are template parameters; wider ones (up to
// 16) run one channel per thread with the taps right-aligned in a window of 16.
#include <string>

#include "attention_kernels.h"
#include "mfma.h"

namespace dm {

constexpr int kCv1Threads = 256;
constexpr int kCv1MaxK = 16;
constexpr int kCv1Batch = 8;     // forward: steps whose loads are issued together
constexpr int kCv1BatchBwd = 4;  // backward: the same (its windows and sums take more registers)

struct Cv1Args {
    int64_t rows;       // B * T (a sequence per batch row) or T (packed)
    int64_t t;          // steps per batch row
    int64_t c, k;       // channels, kernel width
    int64_t nseq;       // sequences S
    const int32_t *cu;  // packed boundaries [S + 1], or null
    int64_t w;          // initial states' steps (with has_h0)
    int64_t w_out;      // final states' steps (with the final states)
    int32_t has_h0, has_bias, silu;
    int64_t seg_len;    // steps per segment
    int64_t cv;         // channel vectors per row
    int64_t nseg;       // segments: the launch's first grid rows
    // the per-sequence work the launch also carries (the forward's final states, the backward's
    // initial states' gradient): aux_blocks blocks of it in aux_rows grid rows after the
    // segments' (a grid-stride loop over the blocks beyond aux_rows x the grid's width)
    int64_t aux_blocks, aux_rows;
};

// The sequence holding row r: s and its rows [s0, s1) (packed: the last sequence whose start is
// at or before r with a nonempty span; empty sequences are stepped over).
__device__ __forceinline__ void cv1_seq(const Cv1Args &a, int64_t r, int64_t *s, int64_t *s0,
                                        int64_t *s1) {
    if (!a.cu) {
        *s = r / a.t;
        *s0 = *s * a.t;
        *s1 = *s0 + a.t;
        return;
    }
    int64_t lo = 0, hi = a.nseq - 1;  // the first s with cu[s + 1] > r
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if ((int64_t)a.cu[mid + 1] > r)
            hi = mid;
        else
            lo = mid + 1;
    }
    *s = lo;
    *s0 = a.cu[lo];
    *s1 = a.cu[lo + 1];
}

__device__ __forceinline__ void cv1_next(const Cv1Args &a, int64_t *s, int64_t *s0, int64_t *s1) {
    ++*s;
    *s0 = *s1;
    *s1 = a.cu ? (int64_t)a.cu[*s + 1] : *s0 + a.t;
}

// VEC consecutive elements of dtype DT at element i, as f32 (16-byte loads when VEC > 1)
template <int DT, int VEC>
__device__ __forceinline__ void cv1_ld(const void *p, int64_t i, float *v) {
    if constexpr (VEC == 1) {
        v[0] = ld<DT>(p, i);
    } else if constexpr (DT == DM_F32) {
#pragma unroll
        for (int q = 0; q < VEC / 4; q++) {
            const float4 a = *(const float4 *)((const float *)p + i + 4 * q);
            v[4 * q] = a.x;
            v[4 * q + 1] = a.y;
            v[4 * q + 2] = a.z;
            v[4 * q + 3] = a.w;
        }
    } else if constexpr (VEC == 4) {
        const uint2 a = *(const uint2 *)((const uint16_t *)p + i);
        const uint32_t u[2] = {a.x, a.y};
#pragma unroll
        for (int e = 0; e < 2; e++) {
            v[2 * e] = unpack_lo<DT>(u[e]);
            v[2 * e + 1] = unpack_hi<DT>(u[e]);
        }
    } else {
        // (non-temporal: the rows stream past once)
        const u32x4_t a = __builtin_nontemporal_load((const u32x4_t *)((const uint16_t *)p + i));
        const uint32_t u[4] = {a[0], a[1], a[2], a[3]};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            v[2 * e] = unpack_lo<DT>(u[e]);
            v[2 * e + 1] = unpack_hi<DT>(u[e]);
        }
    }
}

// the same for f32 states, VEC elements (VEC = 8 of a 16-bit dtype: two 16-byte loads)
template <int VEC>
__device__ __forceinline__ void cv1_ld_state(const float *p, int64_t i, float *v) {
    if constexpr (VEC == 1)
        v[0] = p[i];
    else
        cv1_ld<DM_F32, VEC>(p, i, v);
}

// VEC f32 values stored at element i in dtype DT, rounded to nearest even
template <int DT, int VEC>
__device__ __forceinline__ void cv1_st(void *p, int64_t i, const float *v) {
    if constexpr (VEC == 1) {
        st<DT>(p, i, v[0]);
    } else if constexpr (DT == DM_F32) {
#pragma unroll
        for (int q = 0; q < VEC / 4; q++)
            *(float4 *)((float *)p + i + 4 * q) =
                make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
    } else if constexpr (VEC == 4) {
        *(uint2 *)((uint16_t *)p + i) = make_uint2(pack2<DT>(v[0], v[1]), pack2<DT>(v[2], v[3]));
    } else {
        const u32x4_t o = {pack2<DT>(v[0], v[1]), pack2<DT>(v[2], v[3]), pack2<DT>(v[4], v[5]),
                           pack2<DT>(v[6], v[7])};
        __builtin_nontemporal_store(o, (u32x4_t *)((uint16_t *)p + i));
    }
}

// h[tau] of sequence s (rows [s0, ...)), channels c0 .. c0 + VEC: the inputs at tau >= 0, the
// initial state's step W + tau for -W <= tau < 0, zeros before
template <int DT, int VEC>
__device__ __forceinline__ void cv1_hist(const Cv1Args &a, const void *x, const float *h0, int64_t s,
                                         int64_t s0, int64_t tau, int64_t c0, float *v) {
    if (tau >= 0) {
        cv1_ld<DT, VEC>(x, (s0 + tau) * a.c + c0, v);
    } else if (a.has_h0 && tau >= -a.w) {
        cv1_ld_state<VEC>(h0, (s * a.w + a.w + tau) * a.c + c0, v);
    } else {
#pragma unroll
        for (int e = 0; e < VEC; e++) v[e] = 0.f;
    }
}

__device__ __forceinline__ float cv1_sigmoid(float y) { return 1.f / (1.f + expf(-y)); }

// sigmoid(y) for 16-bit inputs: 1 / (1 + 2^(-y log2 e)) on the hardware exponential and
// reciprocal (about an ulp of f32 each, far below the output's rounding)
__device__ __forceinline__ float cv1_sigmoid_fast(float y) {
    return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-1.4426950408889634f * y));
}

// SiLU(y) = y sigmoid(y). For f32 inputs in f64, rounded once: the device's expf is about an
// ulp off, which the f32 conformance bounds (about 1.3 ulp of the largest output) do not leave
// room for; for 16-bit inputs the output's rounding to the dtype dominates and f32 suffices.
template <int DT>
__device__ __forceinline__ float cv1_silu(float y) {
    if constexpr (DT == DM_F32) {
        const double yd = y;
        return (float)(yd / (1.0 + exp(-yd)));
    } else {
        return y * cv1_sigmoid_fast(y);
    }
}

// acc + a b. For f32 inputs with the product and the sum rounded separately, as the
// reference's tensor operations round them (its conformance bounds are about an ulp); for 16-bit
// inputs, whose results are rounded to 8 or 11 bits, one fused multiply-add.
template <int DT>
__device__ __forceinline__ float cv1_madd(float acc, float a, float b) {
    if constexpr (DT == DM_F32)
        return __fadd_rn(acc, __fmul_rn(a, b));
    else
        return fmaf(a, b, acc);
}


// The taps as KT registers per channel: tap j of a kernel of width k < KT sits at KT - k + j, the
// others are zero (so a window of KT steps ending at the current step applies the kernel).
template <int DT, int VEC, int KT>
__device__ __forceinline__ void cv1_taps(const Cv1Args &a, const void *wt, int64_t c0,
                                         float (&wv)[KT][VEC]) {
    const int off = KT - (int)a.k;
#pragma unroll
    for (int j = 0; j < KT; j++)
#pragma unroll
        for (int e = 0; e < VEC; e++)
            wv[j][e] = j >= off ? ld<DT>(wt, (c0 + e) * a.k + (j - off)) : 0.f;
}

// ------------------------------------------------------------------------------------------
// Forward (conv1d/reference.rs:183-268)
// ------------------------------------------------------------------------------------------

// The final states: the last W' steps of each sequence's history, zeros in front where it is
// shorter (reference.rs:183-197). One thread per (sequence, step, channel).
template <int DT>
__device__ __forceinline__ void cv1_final_block(const Cv1Args &a, const void *__restrict__ x,
                                                const float *__restrict__ h0, float *__restrict__ fin,
                                                int64_t blk) {
    const int64_t cb = (a.c + kCv1Threads - 1) / kCv1Threads;
    const int64_t item = blk / cb;
    const int64_t c = (blk % cb) * kCv1Threads + threadIdx.x;
    if (c >= a.c) return;
    const int64_t s = item / a.w_out, i = item % a.w_out;
    int64_t s0, len;
    if (a.cu) {
        s0 = a.cu[s];
        len = a.cu[s + 1] - s0;
    } else {
        s0 = s * a.t;
        len = a.t;
    }
    const int64_t wh = a.has_h0 ? a.w : 0;
    const int64_t hstep = wh + len - a.w_out + i;  // step of the history, from its first
    float v = 0.f;
    if (hstep >= wh)
        v = ld<DT>(x, (s0 + hstep - wh) * a.c + c);
    else if (hstep >= 0)
        v = h0[(s * a.w + hstep) * a.c + c];
    fin[(s * a.w_out + i) * a.c + c] = v;
}

template <int DT, int VEC, int KT>
__global__ __launch_bounds__(kCv1Threads) void conv1d_fwd_kernel(Cv1Args a, const void *__restrict__ x,
                                                                 const void *__restrict__ wt,
                                                                 const void *__restrict__ bias,
                                                                 const float *__restrict__ h0,
                                                                 void *__restrict__ out,
                                                                 float *__restrict__ fin) {
    if ((int64_t)blockIdx.y >= a.nseg) {  // the final states' rows
        for (int64_t b = ((int64_t)blockIdx.y - a.nseg) * gridDim.x + blockIdx.x; b < a.aux_blocks;
             b += a.aux_rows * gridDim.x)
            cv1_final_block<DT>(a, x, h0, fin, b);
        return;
    }
    const int64_t cvi = (int64_t)blockIdx.x * kCv1Threads + threadIdx.x;
    if (cvi >= a.cv) return;
    const int64_t c0 = cvi * VEC;
    const int64_t r0 = (int64_t)blockIdx.y * a.seg_len;
    const int64_t r1 = min(r0 + a.seg_len, a.rows);
    if (r0 >= r1) return;
    float wv[KT][VEC], bv[VEC];
    cv1_taps<DT, VEC, KT>(a, wt, c0, wv);
#pragma unroll
    for (int e = 0; e < VEC; e++) bv[e] = a.has_bias ? ld<DT>(bias, c0 + e) : 0.f;
    int64_t s, s0, s1;
    cv1_seq(a, r0, &s, &s0, &s1);
    for (int64_t r = r0; r < r1;) {
        while (r >= s1) cv1_next(a, &s, &s0, &s1);
        const int64_t pend = min(r1, s1);
        // the KT - 1 steps before r
        float win[KT][VEC];
#pragma unroll
        for (int j = 0; j < KT - 1; j++) cv1_hist<DT, VEC>(a, x, h0, s, s0, r - s0 - (KT - 1) + j, c0, win[j]);
        // one step from the window (win[KT - 1] the step's input): the taps in order, then the
        // bias (reference.rs:94-105); then the window slides
        auto step = [&](int64_t rr) __attribute__((always_inline)) {
            float o[VEC];
#pragma unroll
            for (int e = 0; e < VEC; e++) {
                float y = 0.f;
#pragma unroll
                for (int j = 0; j < KT; j++) y = cv1_madd<DT>(y, wv[j][e], win[j][e]);
                if (a.has_bias) y = __fadd_rn(y, bv[e]);
                if (a.silu) y = cv1_silu<DT>(y);
                o[e] = y;
            }
            cv1_st<DT, VEC>(out, rr * a.c + c0, o);
#pragma unroll
            for (int j = 0; j < KT - 1; j++)
#pragma unroll
                for (int e = 0; e < VEC; e++) win[j][e] = win[j + 1][e];
        };
        if constexpr (DT != DM_F32 && VEC == 8) {
            // 16-bit rows of 8 channels: two register sets of kCv1Batch raw 16-byte loads, the
            // next batch's loads issued before this batch's steps, so a thread always has a
            // batch in flight while it computes
            u32x4_t ra[kCv1Batch], rb[kCv1Batch];
            auto issue = [&](u32x4_t (&buf)[kCv1Batch], int64_t rr) __attribute__((always_inline)) {
#pragma unroll
                for (int u = 0; u < kCv1Batch; u++)
                    buf[u] = __builtin_nontemporal_load(
                        (const u32x4_t *)((const uint16_t *)x + (rr + u) * a.c + c0));
            };
            auto consume = [&](const u32x4_t (&buf)[kCv1Batch], int64_t rr) __attribute__((always_inline)) {
#pragma unroll
                for (int u = 0; u < kCv1Batch; u++) {
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        win[KT - 1][2 * e] = unpack_lo<DT>(buf[u][e]);
                        win[KT - 1][2 * e + 1] = unpack_hi<DT>(buf[u][e]);
                    }
                    step(rr + u);
                }
            };
            if (r + kCv1Batch <= pend) {
                issue(ra, r);
                while (true) {
                    const bool more = r + 2 * kCv1Batch <= pend;
                    if (more) issue(rb, r + kCv1Batch);
                    consume(ra, r);
                    r += kCv1Batch;
                    if (!more) break;
                    const bool more2 = r + 2 * kCv1Batch <= pend;
                    if (more2) issue(ra, r + kCv1Batch);
                    consume(rb, r);
                    r += kCv1Batch;
                    if (!more2) break;
                }
            }
        }
        // kCv1Batch steps at a time: their rows' loads all issued before the first is used
        for (; r + kCv1Batch <= pend; r += kCv1Batch) {
            float xb[kCv1Batch][VEC];
#pragma unroll
            for (int u = 0; u < kCv1Batch; u++) cv1_ld<DT, VEC>(x, (r + u) * a.c + c0, xb[u]);
#pragma unroll
            for (int u = 0; u < kCv1Batch; u++) {
#pragma unroll
                for (int e = 0; e < VEC; e++) win[KT - 1][e] = xb[u][e];
                step(r + u);
            }
        }
        for (; r < pend; r++) {
            cv1_ld<DT, VEC>(x, r * a.c + c0, win[KT - 1]);
            step(r);
        }
    }
}

// ------------------------------------------------------------------------------------------
// Backward (conv1d/reference.rs:270-482)
// ------------------------------------------------------------------------------------------

// dy = go SiLU'(y), SiLU'(y) = s (y (1 - s) + 1) with s = sigmoid(y) (reference.rs:117-134);
// in f64 for f32 inputs, as the forward's SiLU
template <int DT>
__device__ __forceinline__ float cv1_dy(float g, float y, int silu) {
    if (!silu) return g;
    if constexpr (DT == DM_F32) {
        const double yd = y, sg = 1.0 / (1.0 + exp(-yd));
        return (float)((double)g * (sg * (yd * (1.0 - sg) + 1.0)));
    } else {
        const float sg = cv1_sigmoid_fast(y);
        return g * (sg * fmaf(y, 1.f - sg, 1.f));
    }
}

// The initial states' gradient: per (sequence, channel), the padded steps before the first step
// take sum_j weight[j] dy[q - j] (reference.rs:318-325), the state's earlier steps zero, then the
// final states' gradient where the history is short enough to keep state steps (:342-373). A few
// steps per sequence: computed in f64 and rounded once (f32 leaves it about an ulp off, the width
// of its conformance bound).
template <int DT, int GT>
__device__ __forceinline__ void cv1_h0_block(const Cv1Args &a, const void *__restrict__ x,
                                             const void *__restrict__ wt, const void *__restrict__ bias,
                                             const float *__restrict__ h0, const void *__restrict__ go,
                                             const float *__restrict__ gfin, float *__restrict__ gh0,
                                             int64_t blk) {
    const int64_t cb = (a.c + kCv1Threads - 1) / kCv1Threads;
    const int64_t s = blk / cb;
    const int64_t c = (blk % cb) * kCv1Threads + threadIdx.x;
    if (c >= a.c) return;
    int64_t s0, len;
    if (a.cu) {
        s0 = a.cu[s];
        len = a.cu[s + 1] - s0;
    } else {
        s0 = s * a.t;
        len = a.t;
    }
    const int64_t K = a.k, W = a.w;
    const double b = a.has_bias ? (double)ld<DT>(bias, c) : 0.0;
    auto hist = [&](int64_t tau) -> double {
        if (tau >= 0) return ld<DT>(x, (s0 + tau) * a.c + c);
        if (tau >= -W) return h0[(s * W + W + tau) * a.c + c];
        return 0.0;
    };
    auto dy = [&](int64_t t) -> double {
        double y = 0.0;
        for (int64_t j = 0; j < K; j++) y += (double)ld<DT>(wt, c * K + j) * hist(t - (K - 1) + j);
        y += b;
        const double g = ld<GT>(go, (s0 + t) * a.c + c);
        if (!a.silu) return g;
        const double sg = 1.0 / (1.0 + exp(-y));
        return g * (sg * (y * (1.0 - sg) + 1.0));
    };
    const int64_t P = W + len;
    for (int64_t i = 0; i < W; i++) {
        double g = 0.0;
        const int64_t q = i - (W - (K - 1));  // padded step before the first
        if (q >= 0)
            for (int64_t j = 0; j < K; j++) {
                const int64_t t = q - j;
                if (t >= 0 && t < len) g += (double)ld<DT>(wt, c * K + j) * dy(t);
            }
        if (gfin) {
            const int64_t idx = i - (P - a.w_out);
            if (idx >= 0) g += gfin[(s * a.w_out + idx) * a.c + c];
        }
        gh0[(s * W + i) * a.c + c] = (float)g;
    }
}

template <int DT, int GT, int VEC, int KT>
__global__ __launch_bounds__(kCv1Threads) void conv1d_bwd_kernel(
    Cv1Args a, const void *__restrict__ x, const void *__restrict__ wt, const void *__restrict__ bias,
    const float *__restrict__ h0, const void *__restrict__ go, const float *__restrict__ gfin,
    void *__restrict__ gx, float *__restrict__ part, float *__restrict__ gh0) {
    if ((int64_t)blockIdx.y >= a.nseg) {  // the initial states' gradient's rows
        for (int64_t b = ((int64_t)blockIdx.y - a.nseg) * gridDim.x + blockIdx.x; b < a.aux_blocks;
             b += a.aux_rows * gridDim.x)
            cv1_h0_block<DT, GT>(a, x, wt, bias, h0, go, gfin, gh0, b);
        return;
    }
    const int64_t cvi = (int64_t)blockIdx.x * kCv1Threads + threadIdx.x;
    if (cvi >= a.cv) return;
    const int64_t c0 = cvi * VEC;
    const int64_t seg = blockIdx.y;
    const int64_t r0 = seg * a.seg_len;
    const int64_t r1 = min(r0 + a.seg_len, a.rows);
    float wv[KT][VEC], bv[VEC];
    cv1_taps<DT, VEC, KT>(a, wt, c0, wv);
#pragma unroll
    for (int e = 0; e < VEC; e++) bv[e] = a.has_bias ? ld<DT>(bias, c0 + e) : 0.f;
    float aw[KT][VEC], ab[VEC];
#pragma unroll
    for (int e = 0; e < VEC; e++) {
        ab[e] = 0.f;
#pragma unroll
        for (int j = 0; j < KT; j++) aw[j][e] = 0.f;
    }
    const int64_t wh = a.has_h0 ? a.w : 0;
    // the pre-activation gradient of step tau of sequence s from its window
    // the pre-activation gradient from the output's gradient g and the inputs' window
    auto dy_of = [&](const float *g, const float (&xw)[KT][VEC], float *d) {
#pragma unroll
        for (int e = 0; e < VEC; e++) {
            float y = 0.f;
#pragma unroll
            for (int j = 0; j < KT; j++) y = cv1_madd<DT>(y, wv[j][e], xw[j][e]);
            if (a.has_bias) y = __fadd_rn(y, bv[e]);
            d[e] = cv1_dy<DT>(g[e], y, a.silu);
        }
    };
    auto dy_at = [&](int64_t s0, int64_t tau, const float (&xw)[KT][VEC], float *d) {
        float g[VEC];
        cv1_ld<GT, VEC>(go, (s0 + tau) * a.c + c0, g);
        dy_of(g, xw, d);
    };
    if (r0 < r1) {
        int64_t s, s0, s1;
        cv1_seq(a, r0, &s, &s0, &s1);
        for (int64_t r = r0; r < r1;) {
            while (r >= s1) cv1_next(a, &s, &s0, &s1);
            const int64_t p0 = r, p1 = min(r1, s1), len = s1 - s0;
            // the pre-activation gradients of the KT - 1 steps after the piece (zero past the
            // sequence): gwin[i] holds step p1 + i
            float gwin[KT][VEC];
#pragma unroll
            for (int i = 0; i < KT - 1; i++) {
                const int64_t tau = p1 - s0 + i;
                if (tau < len) {
                    float xw[KT][VEC];
#pragma unroll
                    for (int j = 0; j < KT; j++) cv1_hist<DT, VEC>(a, x, h0, s, s0, tau - (KT - 1) + j, c0, xw[j]);
                    dy_at(s0, tau, xw, gwin[i]);
                } else {
#pragma unroll
                    for (int e = 0; e < VEC; e++) gwin[i][e] = 0.f;
                }
            }
            // the inputs' window of the piece's last step: xw[j] = h[t - (KT - 1) + j]
            float xw[KT][VEC];
#pragma unroll
            for (int j = 0; j < KT; j++) cv1_hist<DT, VEC>(a, x, h0, s, s0, p1 - 1 - s0 - (KT - 1) + j, c0, xw[j]);
            const int64_t P = wh + len;
            // step t from its output gradient g and the windows; then both slide one step back
            // (xn: the input entering the window, h[t - KT])
            auto step = [&](int64_t t, const float *g, const float *xn, auto fin_c) __attribute__((always_inline)) {
                constexpr bool FIN = decltype(fin_c)::value;
                float d[VEC];
                dy_of(g, xw, d);
                // dx[t] = sum_j weight[j] dy[t + K - 1 - j], the taps in order (:296-316): with
                // the taps right-aligned at KT, tap slot j reads dy[t + KT - 1 - j], which is d
                // for j = KT - 1 and gwin[KT - 2 - j] before
                float o[VEC];
#pragma unroll
                for (int e = 0; e < VEC; e++) {
                    float acc = 0.f;
#pragma unroll
                    for (int j = 0; j < KT; j++) {
                        if (j < KT - (int)a.k) continue;  // (zero taps)
                        const float dj = j == KT - 1 ? d[e] : gwin[KT - 2 - j][e];
                        acc = cv1_madd<DT>(acc, wv[j][e], dj);
                    }
                    o[e] = acc;
                }
                // the final states' gradient onto the inputs among the history's last W' steps
                if (FIN) {
                    const int64_t idx = wh + (t - s0) - (P - a.w_out);
                    if (idx >= 0) {
                        float f[VEC];
                        cv1_ld_state<VEC>(gfin, (s * a.w_out + idx) * a.c + c0, f);
#pragma unroll
                        for (int e = 0; e < VEC; e++) o[e] = __fadd_rn(o[e], f[e]);
                    }
                }
                cv1_st<DT, VEC>(gx, t * a.c + c0, o);
#pragma unroll
                for (int e = 0; e < VEC; e++) {
                    ab[e] = __fadd_rn(ab[e], d[e]);
#pragma unroll
                    for (int j = 0; j < KT; j++) aw[j][e] = cv1_madd<DT>(aw[j][e], d[e], xw[j][e]);
                }
#pragma unroll
                for (int i = KT - 2; i > 0; i--)
#pragma unroll
                    for (int e = 0; e < VEC; e++) gwin[i][e] = gwin[i - 1][e];
#pragma unroll
                for (int e = 0; e < VEC; e++) gwin[0][e] = d[e];
#pragma unroll
                for (int j = KT - 1; j > 0; j--)
#pragma unroll
                    for (int e = 0; e < VEC; e++) xw[j][e] = xw[j - 1][e];
#pragma unroll
                for (int e = 0; e < VEC; e++) xw[0][e] = xn[e];
            };
            int64_t t = p1 - 1;
            // the steps the final states' gradient reaches (the history's last W'), one at a time
            const int64_t tfin = gfin ? max(p0, s0 + (P - a.w_out) - wh) : p1;
            for (; t >= tfin; t--) {
                float g[VEC], xn[VEC];
                cv1_ld<GT, VEC>(go, t * a.c + c0, g);
                cv1_hist<DT, VEC>(a, x, h0, s, s0, t - s0 - KT, c0, xn);
                step(t, g, xn, std::true_type{});
            }
            // then kCv1BatchBwd steps at a time, their loads (output gradients and entering
            // inputs) all issued before the first step; inputs inside the sequence read directly
            for (; t - (kCv1BatchBwd - 1) >= p0; t -= kCv1BatchBwd) {
                float gb[kCv1BatchBwd][VEC], xn[kCv1BatchBwd][VEC];
#pragma unroll
                for (int u = 0; u < kCv1BatchBwd; u++) cv1_ld<GT, VEC>(go, (t - u) * a.c + c0, gb[u]);
                if (t - (kCv1BatchBwd - 1) - s0 - KT >= 0) {
#pragma unroll
                    for (int u = 0; u < kCv1BatchBwd; u++) cv1_ld<DT, VEC>(x, (t - u - KT) * a.c + c0, xn[u]);
                } else {
#pragma unroll
                    for (int u = 0; u < kCv1BatchBwd; u++) cv1_hist<DT, VEC>(a, x, h0, s, s0, t - u - s0 - KT, c0, xn[u]);
                }
#pragma unroll
                for (int u = 0; u < kCv1BatchBwd; u++) step(t - u, gb[u], xn[u], std::false_type{});
            }
            for (; t >= p0; t--) {
                float g[VEC], xn[VEC];
                cv1_ld<GT, VEC>(go, t * a.c + c0, g);
                cv1_hist<DT, VEC>(a, x, h0, s, s0, t - s0 - KT, c0, xn);
                step(t, g, xn, std::false_type{});
            }
            r = p1;
        }
    }
    // this segment's partial sums of the weight's and the bias's gradients: [seg][C][K + 1]
    const int off = KT - (int)a.k;
#pragma unroll
    for (int e = 0; e < VEC; e++) {
        float *pp = part + (seg * a.c + c0 + e) * (a.k + 1);
#pragma unroll
        for (int j = 0; j < KT; j++)
            if (j >= off) pp[j - off] = aw[j][e];
        pp[a.k] = ab[e];
    }
}

// The weight's and the bias's gradients: the segments' partials summed in segment order.
template <int DT>
__global__ __launch_bounds__(kCv1Threads) void conv1d_bwd_reduce(int64_t nseg, int64_t C, int64_t K,
                                                                 const float *__restrict__ part,
                                                                 void *__restrict__ gw,
                                                                 void *__restrict__ gb) {
    const int64_t i = (int64_t)blockIdx.x * kCv1Threads + threadIdx.x;
    if (i >= C * (K + 1)) return;
    float acc = 0.f;
#pragma unroll 8
    for (int64_t g = 0; g < nseg; g++) acc = __fadd_rn(acc, part[g * C * (K + 1) + i]);
    const int64_t c = i / (K + 1), j = i % (K + 1);
    if (j < K)
        st<DT>(gw, c * K + j, acc);
    else if (gb)
        st<DT>(gb, c, acc);
}

// ------------------------------------------------------------------------------------------
// The decoding step (conv1d/reference.rs:484-520)
// ------------------------------------------------------------------------------------------

// One thread per (row, channel): the state's last K - 1 steps and the token through the taps;
// the next state is the state without its oldest step, then the token (written in ascending
// step order after every read, so it may overwrite the state in place).
template <int DT>
__global__ __launch_bounds__(kCv1Threads) void conv1d_update_kernel(
    int64_t B, int64_t C, int64_t K, int64_t W, int has_bias, int silu, const void *__restrict__ x,
    const void *__restrict__ wt, const void *__restrict__ bias, const float *state, void *__restrict__ out,
    float *next) {
    // the channel from the grid's first index, the row from its second; a row's state offsets in
    // 32 bits (W x C is checked on the host)
    const int c = blockIdx.x * kCv1Threads + threadIdx.x;
    if (c >= C) return;
    const int64_t b = blockIdx.y;
    const int c32 = (int)C, k32 = (int)K, w32 = (int)W;
    const float *sp = state + b * W * C + c;
    float *np = next + b * W * C + c;
    const float xv = ld<DT>(x, b * C + c);
    float y = 0.f;
    for (int j = 0; j < k32; j++) {
        const float v = j < k32 - 1 ? sp[(w32 - (k32 - 1) + j) * c32] : xv;
        y = cv1_madd<DT>(y, v, ld<DT>(wt, (int64_t)c * K + j));
    }
    if (has_bias) y = __fadd_rn(y, ld<DT>(bias, c));
    if (silu) y = cv1_silu<DT>(y);
    st<DT>(out, b * C + c, y);
    for (int t = 0; t < w32; t++) np[t * c32] = t + 1 < w32 ? sp[(t + 1) * c32] : xv;
}

// ------------------------------------------------------------------------------------------
// Host side
// ------------------------------------------------------------------------------------------

static int cv1_check(const dm_conv1d_desc *d, const char *op, bool step) {
    const std::string o(op);
    if (!d) return refuse(o + ": null descriptor");
    if (d->dtype != DM_F32 && d->dtype != DM_BF16 && d->dtype != DM_F16)
        return refuse(o + ": the dtype must be f32, bf16 or f16");
    if (d->k < 1) return refuse(o + ": the kernel width must be at least 1");
    if (d->k > kCv1MaxK)
        return refuse(o + ": kernel widths above " + std::to_string(kCv1MaxK) +
                      " are not implemented, got " + std::to_string(d->k));
    if (d->b < 0 || d->t < 0 || d->c < 0) return refuse(o + ": negative dimensions");
    if (d->activation != DM_ACT_NONE && d->activation != DM_ACT_SILU)
        return refuse(o + ": activation " + std::to_string(d->activation) + " is not implemented");
    if (step) {
        if (d->w + 1 < d->k)
            return refuse(o + ": a state of " + std::to_string(d->w) +
                          " steps cannot feed a kernel of width " + std::to_string(d->k) +
                          "; it needs at least " + std::to_string(d->k - 1));
        return DM_OK;
    }
    if (d->cu_seqlens) {
        if (d->b != 1)
            return refuse(o + ": packed sequences lie along T of a batch of one, got B = " +
                          std::to_string(d->b));
        if (d->nseq < 1) return refuse(o + ": cu_seqlens must hold N + 1 >= 2 offsets");
    }
    if (d->has_initial && d->w + 1 < d->k)
        return refuse(o + ": a initial state of " + std::to_string(d->w) +
                      " steps cannot feed a kernel of width " + std::to_string(d->k) +
                      "; it needs at least " + std::to_string(d->k - 1));
    if (d->has_final && d->w_out < 0) return refuse(o + ": negative final state length");
    return DM_OK;
}

// compute units of the current device (256 on MI355X), read once
static int cv1_cus() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0, n = 0;
        cus = hipGetDevice(&dev) == hipSuccess &&
                      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
                      n > 0
                  ? n
                  : 256;
    }
    return cus;
}

static int64_t cv1_nseq(const dm_conv1d_desc *d) { return d->cu_seqlens ? d->nseq : d->b; }

// the vector width (channels per thread) a call takes: 16 bytes of channels when C divides
// (the backward takes 4 channels per thread of any dtype: its windows, taps and sums hold 4 K + 4
// registers per channel; widths above 8 run one channel per thread)
static int cv1_vec(const dm_conv1d_desc *d, bool bwd = false) {
    const int v = bwd || d->dtype == DM_F32 ? 4 : 8;
    return d->c % v == 0 && d->k <= 8 ? v : 1;
}

static Cv1Args cv1_args(const dm_conv1d_desc *d, bool bwd = false) {
    Cv1Args a{};
    a.rows = d->cu_seqlens ? d->t : d->b * d->t;
    a.t = d->t;
    a.c = d->c;
    a.k = d->k;
    a.nseq = cv1_nseq(d);
    a.cu = d->cu_seqlens;
    a.w = d->has_initial ? d->w : 0;
    a.w_out = d->has_final ? d->w_out : 0;
    a.has_h0 = d->has_initial ? 1 : 0;
    a.has_bias = d->has_bias ? 1 : 0;
    a.silu = d->activation == DM_ACT_SILU ? 1 : 0;
    const int vec = cv1_vec(d, bwd);
    a.cv = (d->c + vec - 1) / vec;
    // segments: three workgroups of 256 threads per compute unit in all (measured on config 6's
    // shape over 1.3-6 workgroups per compute unit, both directions: the backward 331 us at 4.0
    // and 268 us at 3, the forward 193 us at 4 and 182-186 us at 3; at 3.3-3.5 both slow by 7%, as
    // some compute units then hold a fourth; with the forward's two register sets of loads, at
    // 248 registers, the forward measured 167 us at 3, 204 at 2, 191 at 4 and 168 at 6), at most
    // 512 segments of at least 16 steps
    const int64_t gx = (a.cv + kCv1Threads - 1) / kCv1Threads;
    int64_t nseg = 3 * cv1_cus() / std::max<int64_t>(gx, 1);
    nseg = std::min<int64_t>(nseg, 512);
    nseg = std::min<int64_t>(nseg, (a.rows + 15) / 16);
    nseg = std::max<int64_t>(nseg, 1);
    a.seg_len = (a.rows + nseg - 1) / nseg;
    a.nseg = a.rows ? (a.rows + a.seg_len - 1) / a.seg_len : 0;
    return a;
}

static int64_t cv1_nseg(const Cv1Args &a) { return a.nseg; }

// the per-sequence work's blocks, in rows of the launch's width (at most 4096 rows)
static void cv1_aux(Cv1Args &a, int64_t blocks) {
    const int64_t gx = (a.cv + kCv1Threads - 1) / kCv1Threads;
    a.aux_blocks = blocks;
    a.aux_rows = blocks > 0 ? std::min<int64_t>((blocks + gx - 1) / gx, 4096) : 0;
}

// kernel width -> template instance: 1..8 exactly, wider ones in a window of 16
#define CV1_K_SWITCH(K, MACRO, ...)        \
    switch (K) {                           \
        case 1: MACRO(1, __VA_ARGS__); break; \
        case 2: MACRO(2, __VA_ARGS__); break; \
        case 3: MACRO(3, __VA_ARGS__); break; \
        case 4: MACRO(4, __VA_ARGS__); break; \
        case 5: MACRO(5, __VA_ARGS__); break; \
        case 6: MACRO(6, __VA_ARGS__); break; \
        case 7: MACRO(7, __VA_ARGS__); break; \
        case 8: MACRO(8, __VA_ARGS__); break; \
        default: MACRO(16, __VA_ARGS__); break; \
    }

template <int DT>
static void cv1_fwd_launch(const Cv1Args &a, int vec, const void *x, const void *w, const void *bias,
                           const float *h0, void *out, float *fin, hipStream_t st) {
    const dim3 grid((unsigned)((a.cv + kCv1Threads - 1) / kCv1Threads), (unsigned)(a.nseg + a.aux_rows));
    constexpr int V = DT == DM_F32 ? 4 : 8;
#define CV1_FWD(KT, VV) \
    conv1d_fwd_kernel<DT, VV, KT><<<grid, kCv1Threads, 0, st>>>(a, x, w, bias, h0, out, fin)
    if (vec == V && a.k <= 8) {
        CV1_K_SWITCH(a.k, CV1_FWD, V)
    } else {
        CV1_K_SWITCH(a.k, CV1_FWD, 1)
    }
#undef CV1_FWD
}

template <int DT, int GT>
static void cv1_bwd_launch(const Cv1Args &a, int vec, const void *x, const void *w, const void *bias,
                           const float *h0, const void *go, const float *gfin, void *gx, float *part,
                           float *gh0, hipStream_t st) {
    const dim3 grid((unsigned)((a.cv + kCv1Threads - 1) / kCv1Threads), (unsigned)(a.nseg + a.aux_rows));
    constexpr int V = 4;
#define CV1_BWD(KT, VV)                                                                          \
    conv1d_bwd_kernel<DT, GT, VV, KT><<<grid, kCv1Threads, 0, st>>>(a, x, w, bias, h0, go, gfin, gx, \
                                                                    part, gh0)
    if (vec == V && a.k <= 8) {
        CV1_K_SWITCH(a.k, CV1_BWD, V)
    } else {
        CV1_K_SWITCH(a.k, CV1_BWD, 1)
    }
#undef CV1_BWD
}

}  // namespace dm

using namespace dm;

extern "C" {

int dm_causal_conv1d_fwd(const dm_conv1d_desc *d, const void *x, const void *weight,
                         const void *bias, const float *initial_state, void *out,
                         float *final_state, void *stream) {
    const char *op = "causal_conv1d";
    if (int rc = cv1_check(d, op, false)) return rc;
    if (d->has_bias && !bias) return refuse(std::string(op) + ": has_bias without a bias");
    if (d->has_initial && !initial_state)
        return refuse(std::string(op) + ": has_initial without initial states");
    if (d->has_final && !final_state)
        return refuse(std::string(op) + ": has_final without a final state buffer");
    hipStream_t st = (hipStream_t)stream;
    Cv1Args a = cv1_args(d);
    const int vec = cv1_vec(d);
    // the final states ride in the same launch, as rows after the segments'
    if (d->has_final && a.w_out > 0 && a.nseq > 0 && a.c > 0)
        cv1_aux(a, a.nseq * a.w_out * ((a.c + kCv1Threads - 1) / kCv1Threads));
    {
        KernelTimer timer(DM_KERNEL_CONV1D_FWD, st);
        if (a.c > 0 && a.nseg + a.aux_rows > 0) {
            if (d->dtype == DM_F32)
                cv1_fwd_launch<DM_F32>(a, vec, x, weight, bias, initial_state, out, final_state, st);
            else if (d->dtype == DM_BF16)
                cv1_fwd_launch<DM_BF16>(a, vec, x, weight, bias, initial_state, out, final_state, st);
            else
                cv1_fwd_launch<DM_F16>(a, vec, x, weight, bias, initial_state, out, final_state, st);
        }
    }
    probe_add(DM_PROBE_CONV1D_FWD);
    DM_LAUNCH_CHECK("causal_conv1d: launch");
    return DM_OK;
}

size_t dm_causal_conv1d_bwd_workspace(const dm_conv1d_desc *d) {
    if (!d || d->k < 1 || d->c < 0) return 0;
    const Cv1Args a = cv1_args(d, true);
    return align_up((size_t)std::max<int64_t>(cv1_nseg(a), 1) * (size_t)d->c * (size_t)(d->k + 1) *
                    sizeof(float));
}

int dm_causal_conv1d_bwd(const dm_conv1d_desc *d, const void *x, const void *weight,
                         const void *bias, const float *initial_state, const void *grad_out,
                         int grad_out_dtype, const float *grad_final_state, void *grad_x,
                         void *grad_weight, void *grad_bias, float *grad_initial_state,
                         void *workspace, size_t workspace_bytes, void *stream) {
    const char *op = "causal_conv1d_backward";
    if (int rc = cv1_check(d, op, false)) return rc;
    if (grad_out_dtype != DM_F32 && grad_out_dtype != d->dtype)
        return refuse(std::string(op) + ": the output's gradient is f32 or the inputs' dtype");
    if (d->has_bias && (!bias || !grad_bias))
        return refuse(std::string(op) + ": has_bias without the bias or its gradient");
    if (d->has_initial && (!initial_state || !grad_initial_state))
        return refuse(std::string(op) + ": has_initial without the states or their gradient");
    if (workspace_bytes < dm_causal_conv1d_bwd_workspace(d))
        return refuse(std::string(op) +
                      ": the workspace is smaller than dm_causal_conv1d_bwd_workspace");
    hipStream_t st = (hipStream_t)stream;
    Cv1Args a = cv1_args(d, true);
    const int vec = cv1_vec(d, true);
    // the initial states' gradient rides in the same launch, as rows after the segments'
    if (d->has_initial && a.w > 0 && a.nseq > 0 && a.c > 0)
        cv1_aux(a, a.nseq * ((a.c + kCv1Threads - 1) / kCv1Threads));
    const float *gfin = d->has_final && a.w_out > 0 ? grad_final_state : nullptr;
    float *part = (float *)workspace;
    const int64_t nseg = cv1_nseg(a);
    {
        KernelTimer timer(DM_KERNEL_CONV1D_BWD, st);
        if (a.c > 0 && nseg + a.aux_rows > 0) {
#define CV1_BWD_ARGS a, vec, x, weight, bias, initial_state, grad_out, gfin, grad_x, part, grad_initial_state, st
#define CV1_BWD_DT(DT)                                   \
    if (grad_out_dtype == DM_F32)                        \
        cv1_bwd_launch<DT, DM_F32>(CV1_BWD_ARGS);        \
    else                                                 \
        cv1_bwd_launch<DT, DT>(CV1_BWD_ARGS)
            if (d->dtype == DM_F32) {
                cv1_bwd_launch<DM_F32, DM_F32>(CV1_BWD_ARGS);
            } else if (d->dtype == DM_BF16) {
                CV1_BWD_DT(DM_BF16);
            } else {
                CV1_BWD_DT(DM_F16);
            }
#undef CV1_BWD_ARGS
#undef CV1_BWD_DT
        }
    }
    if (a.c > 0) {
        const int64_t n = a.c * (a.k + 1);
        const unsigned blocks = (unsigned)((n + kCv1Threads - 1) / kCv1Threads);
        void *gb = d->has_bias ? grad_bias : nullptr;
        if (nseg == 0) {
            // no steps at all: the weight's and the bias's gradients are zero
            fill_zero(grad_weight, (size_t)(a.c * a.k) * dtype_bytes(d->dtype), st);
            if (gb) fill_zero(gb, (size_t)a.c * dtype_bytes(d->dtype), st);
        } else if (d->dtype == DM_F32) {
            conv1d_bwd_reduce<DM_F32><<<blocks, kCv1Threads, 0, st>>>(nseg, a.c, a.k, part, grad_weight, gb);
        } else if (d->dtype == DM_BF16) {
            conv1d_bwd_reduce<DM_BF16><<<blocks, kCv1Threads, 0, st>>>(nseg, a.c, a.k, part, grad_weight, gb);
        } else {
            conv1d_bwd_reduce<DM_F16><<<blocks, kCv1Threads, 0, st>>>(nseg, a.c, a.k, part, grad_weight, gb);
        }
    }
    probe_add(DM_PROBE_CONV1D_BWD);
    DM_LAUNCH_CHECK("causal_conv1d_backward: launch");
    return DM_OK;
}

int dm_causal_conv1d_update(const dm_conv1d_desc *d, const void *x, const void *weight,
                            const void *bias, const float *state, void *out, float *next_state,
                            void *stream) {
    const char *op = "causal_conv1d_update";
    if (int rc = cv1_check(d, op, true)) return rc;
    if (d->has_bias && !bias) return refuse(std::string(op) + ": has_bias without a bias");
    if (d->w * d->c >= (1ll << 31))
        return refuse(std::string(op) + ": a row's state of 2^31 or more values is not implemented");
    hipStream_t st = (hipStream_t)stream;
    const int64_t n = d->b * d->c;
    if (n > 0) {
        KernelTimer timer(DM_KERNEL_CONV1D_UPDATE, st);
        const int silu = d->activation == DM_ACT_SILU;
        const size_t xb = dtype_bytes(d->dtype);
        // the rows in launches of at most 65535 (the grid's second index)
        for (int64_t b0 = 0; b0 < d->b; b0 += 65535) {
            const int64_t nb = std::min<int64_t>(65535, d->b - b0);
            const dim3 blocks((unsigned)((d->c + kCv1Threads - 1) / kCv1Threads), (unsigned)nb);
            const void *xr = (const char *)x + (size_t)(b0 * d->c) * xb;
            void *outr = (char *)out + (size_t)(b0 * d->c) * xb;
            const float *sr = state + b0 * d->w * d->c;
            float *nr = next_state + b0 * d->w * d->c;
#define CV1_UPD(DT)                                                                              \
    conv1d_update_kernel<DT><<<blocks, kCv1Threads, 0, st>>>(nb, d->c, d->k, d->w, d->has_bias, \
                                                             silu, xr, weight, bias, sr, outr,   \
                                                             nr)
            if (d->dtype == DM_F32) {
                CV1_UPD(DM_F32);
            } else if (d->dtype == DM_BF16) {
                CV1_UPD(DM_BF16);
            } else {
                CV1_UPD(DM_F16);
            }
#undef CV1_UPD
        }
    }
    probe_add(DM_PROBE_CONV1D_UPDATE);
    DM_LAUNCH_CHECK("causal_conv1d_update: launch");
    return DM_OK;
}

}  // extern "C"
