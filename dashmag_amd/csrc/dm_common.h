// Shared device and host helpers of the dashmi kernels: dtype conversion, wave reductions,
// launch probes, refusals, and the attention visibility intervals (bit-exact integer work).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <cmath>
#include <string>

#include "../../include/dashmi.h"

namespace dm {

// ------------------------------------------------------------------------------------------
// Refusals and errors
// ------------------------------------------------------------------------------------------

void set_error(const std::string &msg);
int refuse(const std::string &msg);  // sets the message, returns DM_ERR_REFUSED
int hip_status(hipError_t e, const char *what);
void probe_add(int probe, uint64_t n = 1);

// Records a HIP event pair around the launches in its scope while kernel timing is enabled
// (dm_kernel_timing); does nothing otherwise.
class KernelTimer {
  public:
    KernelTimer(int kernel, hipStream_t stream);
    ~KernelTimer();

  private:
    int kernel_;
    hipStream_t stream_;
    hipEvent_t start_ = nullptr;
};
bool device_ok(std::string *why);

#define DM_LAUNCH_CHECK(what)                                                   \
    do {                                                                        \
        hipError_t e__ = hipGetLastError();                                     \
        if (e__ != hipSuccess) return ::dm::hip_status(e__, what);              \
    } while (0)

// ------------------------------------------------------------------------------------------
// Element access by dtype: f32, bf16 (round to nearest even) and f16
// ------------------------------------------------------------------------------------------

__host__ __device__ inline float bf16_to_f32(uint16_t x) {
    union {
        uint32_t u;
        float f;
    } v;
    v.u = (uint32_t)x << 16;
    return v.f;
}

__host__ __device__ inline uint16_t f32_to_bf16(float f) {
    union {
        uint32_t u;
        float f;
    } v;
    v.f = f;
    uint32_t u = v.u;
    if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u >> 16) | ((u & 0xffff) ? 0x40 : 0));
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

template <int DT>
__device__ __forceinline__ float ld(const void *p, int64_t i);
template <>
__device__ __forceinline__ float ld<DM_F32>(const void *p, int64_t i) {
    return ((const float *)p)[i];
}
template <>
__device__ __forceinline__ float ld<DM_BF16>(const void *p, int64_t i) {
    return bf16_to_f32(((const uint16_t *)p)[i]);
}
template <>
__device__ __forceinline__ float ld<DM_F16>(const void *p, int64_t i) {
    return (float)((const _Float16 *)p)[i];
}

template <int DT>
__device__ __forceinline__ void st(void *p, int64_t i, float x);
template <>
__device__ __forceinline__ void st<DM_F32>(void *p, int64_t i, float x) {
    ((float *)p)[i] = x;
}
template <>
__device__ __forceinline__ void st<DM_BF16>(void *p, int64_t i, float x) {
    ((uint16_t *)p)[i] = f32_to_bf16(x);
}
template <>
__device__ __forceinline__ void st<DM_F16>(void *p, int64_t i, float x) {
    ((_Float16 *)p)[i] = (_Float16)x;
}

// A load by a dtype known only at run time (g and beta may be f32 or the inputs' dtype).
__device__ __forceinline__ float ld_any(int dt, const void *p, int64_t i) {
    if (dt == DM_F32) return ((const float *)p)[i];
    if (dt == DM_BF16) return bf16_to_f32(((const uint16_t *)p)[i]);
    return (float)((const _Float16 *)p)[i];
}
__device__ __forceinline__ void st_any(int dt, void *p, int64_t i, float x) {
    if (dt == DM_F32)
        ((float *)p)[i] = x;
    else if (dt == DM_BF16)
        ((uint16_t *)p)[i] = f32_to_bf16(x);
    else
        ((_Float16 *)p)[i] = (_Float16)x;
}

// ------------------------------------------------------------------------------------------
// Wave64 reductions
// ------------------------------------------------------------------------------------------

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
    return x;
}

// ------------------------------------------------------------------------------------------
// Which keys a query sees (crates/dash-contract/src/attention.rs:33-58)
// ------------------------------------------------------------------------------------------

// The mask as the kernels take it: window sides already resolved (causality as right = 0, a
// side that cannot bind within span = Tq + Tk + 1 as -1, as the reference's `bound` does,
// reference.rs:77-79).
struct MaskInfo {
    int32_t kind;
    int64_t tq, tk;
    int64_t left, right;  // -1: unbounded
    const uint8_t *pad;   // [B, Tk]
    const int32_t *cu_q, *cu_k;
    int32_t nseq;
};

// The sequence holding position `at` among `n` sequences cut by `cu`: the number of ends
// cu[1..n] at or before it, clamped into 0..n-1 (reference.rs:118-159), by binary search.
__host__ __device__ inline int32_t sequence_of(const int32_t *cu, int32_t n, int64_t at) {
    int32_t lo = 0, hi = n;  // count of ends <= at lies in [lo, hi]
    while (lo < hi) {
        int32_t mid = (lo + hi + 1) >> 1;  // is cu[mid] <= at ?
        if ((int64_t)cu[mid] <= at)
            lo = mid;
        else
            hi = mid - 1;
    }
    return lo > n - 1 ? n - 1 : lo;
}

// The interval [lo, hi) of keys query i sees, before key padding. Packed queries outside every
// sequence, and every query of an empty mask, see none (lo = hi = 0).
__host__ __device__ inline void row_bounds(const MaskInfo &m, int64_t i, int64_t *lo,
                                           int64_t *hi) {
    int64_t pos, base, len;
    if (m.kind == DM_MASK_PACKED) {
        int32_t n = m.nseq;
        if (n <= 0 || m.tq == 0 || m.tk == 0 || i < m.cu_q[0] || i >= m.cu_q[n]) {
            *lo = *hi = 0;
            return;
        }
        int32_t s = sequence_of(m.cu_q, n, i);
        int64_t qs = m.cu_q[s], ql = (int64_t)m.cu_q[s + 1] - qs;
        base = m.cu_k[s];
        len = (int64_t)m.cu_k[s + 1] - base;
        pos = (i - qs) + len - ql;
        int64_t a = 0, b = len;
        if (m.right >= 0 && pos + m.right + 1 < b) b = pos + m.right + 1;
        if (m.left >= 0 && pos - m.left > a) a = pos - m.left;
        // offsets past the keys (malformed, outside the contract) never index out of bounds
        a += base;
        b += base;
        if (a < 0) a = 0;
        if (b > m.tk) b = m.tk;
        if (a >= b) a = b = 0;
        *lo = a;
        *hi = b;
        return;
    }
    pos = i + m.tk - m.tq;
    int64_t a = 0, b = m.tk;
    if (m.right >= 0 && pos + m.right + 1 < b) b = pos + m.right + 1;
    if (m.left >= 0 && pos - m.left > a) a = pos - m.left;
    if (a >= b) a = b = 0;
    *lo = a;
    *hi = b;
}

// Builds the kernels' mask from a call's descriptor.
inline MaskInfo mask_info(const dm_attention_desc *d) {
    MaskInfo m;
    m.kind = d->mask_kind;
    m.tq = d->tq;
    m.tk = d->tk;
    const uint64_t span = (uint64_t)(d->tq + d->tk + 1);
    const dm_attention_options &o = d->options;
    uint64_t left = o.has_window ? o.window_left : DM_UNBOUNDED;
    uint64_t right = o.causal ? 0 : (o.has_window ? o.window_right : DM_UNBOUNDED);
    m.left = left < span ? (int64_t)left : -1;
    m.right = right < span ? (int64_t)right : -1;
    m.pad = d->key_padding;
    m.cu_q = d->cu_seqlens_q;
    m.cu_k = d->cu_seqlens_k;
    m.nseq = (int32_t)d->nseq;
    return m;
}

inline float scale_of(const dm_attention_desc *d) {
    return d->options.has_scale ? d->options.scale : (float)(1.0 / std::sqrt((double)d->d));
}

inline size_t align_up(size_t x, size_t a = 256) { return (x + a - 1) / a * a; }

// Element strides of an input along (batch, time, head); the last dimension is contiguous.
struct Strd {
    int64_t b, t, h;
};
// The attention inputs' strides: q, k, v, and the backward's o and d_o (g). Contiguous
// [B, T, H, D] unless the descriptor gives others.
struct AttnStrides {
    Strd q, k, v, o, g;
};

inline AttnStrides attn_strides(const dm_attention_desc *d) {
    const Strd cq{d->tq * d->hq * d->d, d->hq * d->d, d->d};
    const Strd ck{d->tk * d->hkv * d->d, d->hkv * d->d, d->d};
    AttnStrides s{cq, ck, ck, cq, cq};
    if (d->strided) {
        auto cv = [](const dm_strides &x) { return Strd{x.b, x.t, x.h}; };
        s = AttnStrides{cv(d->sq), cv(d->sk), cv(d->sv), cv(d->so), cv(d->sdo)};
    }
    return s;
}

inline bool strides_ok(const Strd &x) { return x.b >= 0 && x.t >= 0 && x.h >= 0; }
// 16-byte rows for the 16-bit kernels' vector loads: every stride a multiple of 8 elements
inline bool strides_16b(const Strd &x) { return x.b % 8 == 0 && x.t % 8 == 0 && x.h % 8 == 0; }
inline bool aligned_16b(const void *p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace dm
