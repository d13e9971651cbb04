// The chosen-token log-probability and entropy under a large vocabulary, with the gradient of
// each row's log-probability for its hidden row (crates/dash-contract/src/logprob.rs:1-56,
// crates/dash-ops/src/logprob.rs:1-56, logprob/reference.rs:64-287).
//
// For a block of rows and a chunk of C vocabulary tokens:
//   1. Z [rows, C] f32 = hidden · weight_cᵀ, one library GEMM (hipBLASLt, bf16 operands with f32
//      accumulation, or f32 throughout): the logits are never held for more than one chunk;
//   2. lp_stats, one workgroup per row: the masked online log-sum-exp of the chunk (running
//      maximum m, s = Σ e^{z-m}, a = Σ e^{z-m}(z-m) for the entropy, r = s without the target's
//      term, the target's logit), and, with the gradient, the row of o rescaled by e^{m_old-m_new}
//      and the softmax weights e^{z-m} of the non-target unmasked tokens written for the next
//      product, as a bf16 part and a bf16 remainder (16 significant bits; each product of two
//      bf16 numbers is exact in f32) or in f32;
//   3. o [rows, D] += E · weight_c, two accumulating GEMMs (the part and the remainder) or one
//      in f32.
// lp_finish then gives logprob = z_t - (m + ln s) (-inf without an unmasked target in range),
// entropy = ln s - a / s and grad = (r weight[t] - o) / s, o accumulated in the gradient's own
// buffer. Row blocks and chunk sizes follow LogprobOptions (logprob.rs:90-111): they set what
// is held at once and the order of the sums.
//
// Roofline: two GEMMs of 2 n V D flops each (one without the gradient; the remainder's GEMM is a
// third), bound by MFMA; lp_stats moves 12 bytes per logit (Z read, E written as two bf16 parts).
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <functional>
#include <map>
#include <string>
#include <vector>

#include "attention_kernels.h"
#include "dm_common.h"
#include "mfma.h"

namespace dm {

enum { LP_M = 0, LP_S, LP_R, LP_A, LP_ZT, LP_FOUND, LP_ZSUM, LP_NSTATE };

constexpr int kLpThreads = 256;
constexpr int64_t kLpMaxChunk = 8192;  // 1024 columns per register group, 8 groups

__device__ __forceinline__ bool lp_masked(const uint32_t *bits, int64_t tok) {
    return (bits[tok >> 5] >> (tok & 31)) & 1u;
}

// Sum and maximum over the workgroup's 4 wavefronts, in a fixed order.
__device__ __forceinline__ float lp_block_sum(float x, float *sm) {
    x = wave_sum(x);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sm[w] = x;
    __syncthreads();
    return (sm[0] + sm[1]) + (sm[2] + sm[3]);
}
__device__ __forceinline__ float lp_block_max(float x, float *sm) {
    x = wave_max(x);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sm[w] = x;
    __syncthreads();
    return fmaxf(fmaxf(sm[0], sm[1]), fmaxf(sm[2], sm[3]));
}

// State per row: m = f32::MIN (so that m_old - m_new is never inf - inf), the sums 0
// (reference.rs:229-240); the gradient's accumulator rows zeroed.
__global__ __launch_bounds__(kLpThreads) void lp_init(int64_t rows, int64_t D, float *st,
                                                      int64_t nst, float *o) {
    const int64_t row = blockIdx.x;
    if (row >= rows) return;
    if (threadIdx.x < LP_NSTATE) st[threadIdx.x * nst + row] = threadIdx.x == LP_M ? -FLT_MAX : 0.f;
    if (o)
        for (int64_t e = threadIdx.x; e < D; e += kLpThreads) o[row * D + e] = 0.f;
}

// One row's statistics for one chunk, each logit read once: thread t holds columns
// 4 t + 1024 i + q (i < NV, q < 4) in registers (16-byte loads when the chunk width is a multiple
// of 4), so a chunk of up to 1024 NV columns is read from memory once. `bits` holds the masked
// words of the vocabulary (bit j of word j / 32 set for a masked token).
// EK: 0 no gradient, 1 the weights as bf16 part + remainder, 2 the weights in f32.
template <int EK, int NV>
__global__ __launch_bounds__(kLpThreads) void lp_stats(int64_t rows, int64_t cw, int64_t c0,
                                                       int64_t D, const float *__restrict__ Z,
                                                       const int64_t *__restrict__ targets,
                                                       const uint32_t *__restrict__ bits,
                                                       float *__restrict__ st, int64_t nst,
                                                       void *__restrict__ E, void *__restrict__ E2,
                                                       float *__restrict__ o) {
    __shared__ float sm[4];
    const int64_t row = blockIdx.x;
    if (row >= rows) return;
    const float *z = Z + row * cw;
    const bool vec = (cw & 3) == 0;
    float x[NV][4];
    uint32_t live = 0;  // bit 4 i + q: column 4 t + 1024 i + q is in the chunk and unmasked
    // the chunk's maximum over the unmasked tokens
    float mx = -FLT_MAX;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int64_t j = 4 * (int64_t)threadIdx.x + 1024 * i;
        if (vec && j < cw) {
            const float4 v = *(const float4 *)(z + j);
            x[i][0] = v.x, x[i][1] = v.y, x[i][2] = v.z, x[i][3] = v.w;
        } else {
#pragma unroll
            for (int q = 0; q < 4; q++) x[i][q] = j + q < cw ? z[j + q] : -FLT_MAX;
        }
        // the masked bits of the 4 columns: one word when they share it
        const int64_t tok = c0 + j;
        uint32_t mb = 0;
        if (j < cw) {
            if ((tok & 31) <= 28) {
                mb = bits[tok >> 5] >> (tok & 31);
            } else {
#pragma unroll
                for (int q = 0; q < 4; q++)
                    if (j + q < cw) mb |= (uint32_t)lp_masked(bits, tok + q) << q;
            }
        }
#pragma unroll
        for (int q = 0; q < 4; q++)
            if (j + q < cw && !((mb >> q) & 1u)) {
                live |= 1u << (4 * i + q);
                mx = fmaxf(mx, x[i][q]);
            }
    }
    mx = lp_block_max(mx, sm);
    // this row's running state, read by every thread before the block reductions below (thread
    // 0 rewrites it after them)
    const float m = st[LP_M * nst + row];
    const float s_old = st[LP_S * nst + row], a_old = st[LP_A * nst + row];
    const float r_old = st[LP_R * nst + row];
    const float m_new = mx > m ? mx : m;
    const float shift = m - m_new, alpha = expf(shift);
    const int64_t t = targets[row];
    const int64_t tl = t - c0;
    const bool has_t = tl >= 0 && tl < cw && !lp_masked(bits, t);
    // the chunk's sums; the weights of the next product (0 for the target and masked tokens)
    float se = 0.f, sa = 0.f, sr = 0.f, sz = 0.f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int64_t j = 4 * (int64_t)threadIdx.x + 1024 * i;
        if (j >= cw) continue;
        float e[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            e[q] = 0.f;
            if ((live >> (4 * i + q)) & 1u) {
                const float dz = x[i][q] - m_new;
                e[q] = expf(dz);
                se += e[q];
                sa += e[q] * dz;
                sz += x[i][q];
                if (j + q == tl) e[q] = 0.f;
                sr += e[q];
            }
        }
        if constexpr (EK == 1) {
            uint16_t hi[4], lo[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                hi[q] = f32_to_bf16(e[q]);
                lo[q] = f32_to_bf16(e[q] - bf16_to_f32(hi[q]));
            }
            uint16_t *eh = (uint16_t *)E + row * cw + j, *el = (uint16_t *)E2 + row * cw + j;
            if (vec) {
                *(uint2 *)eh = make_uint2(hi[0] | (uint32_t)hi[1] << 16, hi[2] | (uint32_t)hi[3] << 16);
                *(uint2 *)el = make_uint2(lo[0] | (uint32_t)lo[1] << 16, lo[2] | (uint32_t)lo[3] << 16);
            } else {
#pragma unroll
                for (int q = 0; q < 4; q++)
                    if (j + q < cw) eh[q] = hi[q], el[q] = lo[q];
            }
        } else if constexpr (EK == 2) {
            float *ef = (float *)E + row * cw + j;
            if (vec) {
                *(float4 *)ef = make_float4(e[0], e[1], e[2], e[3]);
            } else {
#pragma unroll
                for (int q = 0; q < 4; q++)
                    if (j + q < cw) ef[q] = e[q];
            }
        }
    }
    se = lp_block_sum(se, sm);
    sz = lp_block_sum(sz, sm);
    sa = lp_block_sum(sa, sm);
    sr = lp_block_sum(sr, sm);
    if constexpr (EK != 0) {
        // o is still zero while nothing has been summed (the first chunk)
        if (alpha != 1.f && s_old != 0.f)
            for (int64_t e = threadIdx.x; e < D; e += kLpThreads) o[row * D + e] *= alpha;
    }
    if (threadIdx.x == 0) {
        st[LP_A * nst + row] = alpha * (a_old + s_old * shift) + sa;
        st[LP_S * nst + row] = s_old * alpha + se;
        st[LP_R * nst + row] = r_old * alpha + sr;
        if (has_t) {
            st[LP_ZT * nst + row] += z[tl];
            st[LP_FOUND * nst + row] += 1.f;
        }
        st[LP_M * nst + row] = m_new;
        st[LP_ZSUM * nst + row] += sz;
    }
}

// logprob, entropy and, with o, the gradient (r found weight[t] - o) / s in o's place
// (reference.rs:96-120).
template <int WT>
__global__ __launch_bounds__(kLpThreads) void lp_finish(int64_t rows, int64_t V, int64_t D,
                                                        const float *__restrict__ st, int64_t nst,
                                                        const int64_t *__restrict__ targets,
                                                        const void *__restrict__ weight,
                                                        float *__restrict__ logprob,
                                                        float *__restrict__ entropy,
                                                        float *__restrict__ o) {
    const int64_t row = blockIdx.x;
    if (row >= rows) return;
    const float m = st[LP_M * nst + row], s = st[LP_S * nst + row], r = st[LP_R * nst + row];
    const float a = st[LP_A * nst + row], zt = st[LP_ZT * nst + row];
    const float found = st[LP_FOUND * nst + row];
    if (threadIdx.x == 0) {
        const float ln_s = logf(s);
        logprob[row] = found > 0.5f ? zt - (m + ln_s) : -INFINITY;
        entropy[row] = ln_s - a / s;
    }
    if (o) {
        const int64_t t = targets[row];
        const bool in_range = t >= 0 && t < V;
        const float coef = r * found;
        for (int64_t e = threadIdx.x; e < D; e += kLpThreads) {
            const float wt = in_range ? ld<WT>(weight, t * D + e) : 0.f;
            o[row * D + e] = (wt * coef - o[row * D + e]) / s;
        }
    }
}

__global__ void lp_widen(int64_t count, const uint16_t *__restrict__ x, float *__restrict__ y) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (int64_t)gridDim.x * blockDim.x)
        y[i] = bf16_to_f32(x[i]);
}

// ------------------------------------------------------------------------------------------
// The fused linear cross-entropy (crates/dash-contract/src/loss.rs; crates/dash-ops/src/loss.rs)
// ------------------------------------------------------------------------------------------

enum { LCE_LOSS = 0, LCE_LOGPROB, LCE_ENTROPY, LCE_LSE, LCE_Q, LCE_S, LCE_COUNTED, LCE_FOUND };
enum { LC_A = 0, LC_T, LC_E, LC_C, LC_COUNT };

// The rows' outputs from the pass's sums (loss.rs:456-525 finish): rows [8, n] = loss, logprob,
// entropy (0 on an ignored row), lse, q = r / s (1 - p(target)), s, counted, found.
__global__ void lce_finish(int64_t n, const float *__restrict__ st, const int64_t *__restrict__ targets,
                           int64_t ignore_index, float eps, float lam, float inv_classes,
                           float *__restrict__ rows) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float m = st[LP_M * n + i], s = st[LP_S * n + i], r = st[LP_R * n + i];
    const float a = st[LP_A * n + i], zt = st[LP_ZT * n + i], zsum = st[LP_ZSUM * n + i];
    const bool seen = st[LP_FOUND * n + i] > 0.5f, counted = targets[i] != ignore_index;
    const float ln_s = logf(s), lse = m + ln_s;
    float loss = 0.f;
    if (eps < 1.f) loss = (1.f - eps) * (seen ? lse - zt : INFINITY);
    if (eps != 0.f) loss += eps * (lse - zsum * inv_classes);
    if (lam != 0.f) loss += lam * (lse * lse);
    rows[LCE_LOSS * n + i] = counted ? loss : 0.f;
    rows[LCE_LOGPROB * n + i] = counted ? (seen ? zt - lse : -INFINITY) : 0.f;
    rows[LCE_ENTROPY * n + i] = counted ? ln_s - a / s : 0.f;
    rows[LCE_LSE * n + i] = lse;
    rows[LCE_Q * n + i] = r / s;
    rows[LCE_S * n + i] = s;
    rows[LCE_COUNTED * n + i] = counted ? 1.f : 0.f;
    rows[LCE_FOUND * n + i] = seen ? 1.f : 0.f;
}

// The gradient pass's coefficients per row (loss.rs:597-668) from the upstream gradients of the
// loss, logprob and entropy rows (0 on an ignored row): A = gl (1 + 2 lambda lse) - gp - ge H,
// the target's value T + C (T = gl (eps + 2 lambda lse) - q (gl (1 + 2 lambda lse) - gp)
// - (1 - q)(ge H + ge logprob) where found), E = ge (with the entropy), C = -gl eps / K.
__global__ void lce_coef(int64_t n, const float *__restrict__ rows,
                         const float *__restrict__ upstream, float eps, float lam,
                         float inv_classes, int entropy, float *__restrict__ coef) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const bool counted = rows[LCE_COUNTED * n + i] > 0.5f;
    const float gl = counted ? upstream[i] : 0.f, gp = counted ? upstream[n + i] : 0.f;
    const float ge = entropy && counted ? upstream[2 * n + i] : 0.f;
    const float lse = rows[LCE_LSE * n + i], q = rows[LCE_Q * n + i];
    float soft = gl - gp;
    if (lam != 0.f) soft += gl * (lse * 2.f * lam);
    float tgt = -q * soft;
    float glt = gl * eps;
    if (lam != 0.f) glt += gl * (lse * 2.f * lam);
    tgt += glt;
    if (entropy) {
        const float ent = ge * rows[LCE_ENTROPY * n + i];
        soft -= ent;
        const float pt = 1.f - q;
        tgt -= pt * ent + ge * pt * rows[LCE_LOGPROB * n + i];
    }
    const float c = -gl * eps * inv_classes;
    coef[LC_A * n + i] = soft;
    coef[LC_T * n + i] = (rows[LCE_FOUND * n + i] > 0.5f ? tgt : 0.f) + c;
    coef[LC_E * n + i] = ge;
    coef[LC_C * n + i] = c;
}

// The logits' gradient of a chunk (logprob/reference.rs:345-366): g = e^{z - lse}(A - E (z - lse))
// + C, T + C at the target, 0 at a masked id; written as bf16 (BF = true, the products' operand,
// as torch's bf16 linear layer rounds its output's gradient) or f32. One row per workgroup.
template <bool BF>
__global__ __launch_bounds__(kLpThreads) void lce_dz(int64_t rows, int64_t cw, int64_t c0,
                                                     const float *__restrict__ Z,
                                                     const int64_t *__restrict__ targets,
                                                     const uint32_t *__restrict__ bits,
                                                     const float *__restrict__ rowsv,
                                                     const float *__restrict__ coef, int64_t n,
                                                     void *__restrict__ G) {
    const int64_t row = blockIdx.x;
    if (row >= rows) return;
    const float lse = rowsv[LCE_LSE * n + row], A = coef[LC_A * n + row];
    const float T = coef[LC_T * n + row], E = coef[LC_E * n + row], C = coef[LC_C * n + row];
    const int64_t tl = targets[row] - c0;
    const float *z = Z + row * cw;
    for (int64_t j = threadIdx.x; j < cw; j += kLpThreads) {
        float g;
        if (lp_masked(bits, c0 + j)) {
            g = 0.f;
        } else if (j == tl) {
            g = T;
        } else {
            const float dz = z[j] - lse;
            g = expf(dz) * (A - E * dz) + C;
        }
        if constexpr (BF)
            ((uint16_t *)G)[row * cw + j] = f32_to_bf16(g);
        else
            ((float *)G)[row * cw + j] = g;
    }
}

// f32 -> the dtype (a copy for f32), and fills with zeros.
// f32 -> the dtype, 8 elements a thread per pass (two 16-byte loads, one 16-byte store for a
// 16-bit dtype); the tail past a multiple of 8 element by element.
__global__ void lp_cast(int64_t count, const float *__restrict__ x, void *__restrict__ y, int dt) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    // whole 16-byte stores only into a 16-byte aligned destination (a caller's output may be
    // an offset view); element by element otherwise
    const int64_t n8 = ((uintptr_t)y & 15) ? 0 : count / 8;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += stride) {
        const f32x4_t av = __builtin_nontemporal_load((const f32x4_t *)x + 2 * i);
        const f32x4_t bv = __builtin_nontemporal_load((const f32x4_t *)x + 2 * i + 1);
        const float4 a = make_float4(av[0], av[1], av[2], av[3]);
        const float4 b = make_float4(bv[0], bv[1], bv[2], bv[3]);
        if (dt == DM_F32) {
            ((float4 *)y)[2 * i] = a;
            ((float4 *)y)[2 * i + 1] = b;
        } else if (dt == DM_BF16) {
            ((uint4 *)y)[i] = make_uint4(pack2<DM_BF16>(a.x, a.y), pack2<DM_BF16>(a.z, a.w),
                                         pack2<DM_BF16>(b.x, b.y), pack2<DM_BF16>(b.z, b.w));
        } else {
            ((uint4 *)y)[i] = make_uint4(pack2<DM_F16>(a.x, a.y), pack2<DM_F16>(a.z, a.w),
                                         pack2<DM_F16>(b.x, b.y), pack2<DM_F16>(b.z, b.w));
        }
    }
    for (int64_t i = 8 * n8 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += stride)
        st_any(dt, y, i, x[i]);
}
__global__ void lp_zero(int64_t count, float *__restrict__ x) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (int64_t)gridDim.x * blockDim.x)
        x[i] = 0.f;
}
__global__ void lp_widen16(int64_t count, const _Float16 *__restrict__ x, float *__restrict__ y) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (int64_t)gridDim.x * blockDim.x)
        y[i] = (float)x[i];
}

// hipBLASLt: one handle per (thread, device); per GEMM shape, the descriptors and the
// heuristic's first algorithm, kept for the process.
constexpr size_t kLtWorkspace = 64u << 20;  // the library's workspace, part of ours

struct LtGemm {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    bool ok = false;
};

static hipblasLtHandle_t lt_handle() {
    thread_local std::map<int, hipblasLtHandle_t> handles;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    auto it = handles.find(dev);
    if (it == handles.end()) {
        hipblasLtHandle_t h = nullptr;
        if (hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS) return nullptr;
        it = handles.emplace(dev, h).first;
    }
    return it->second;
}

// Column-major D (m x n, ld m) = op(A) op(B) + beta D, f32 out, f32 accumulation; A and B of
// type `t`, A stored m x k (ta = N, lda m) or k x m (ta = T, lda k), B stored k x n (tb = N,
// ldb k) or n x k (tb = T, ldb n).
static int lt_gemm(hipStream_t st, bool ta, bool tb, int64_t m, int64_t n, int64_t k,
                   const void *A, const void *B, hipDataType t, float beta, float *Dm, void *ws) {
    hipblasLtHandle_t h = lt_handle();
    if (!h) {
        set_error("no hipBLASLt handle");
        return DM_ERR_HIP;
    }
    int dev = 0;
    (void)hipGetDevice(&dev);
    thread_local std::map<std::vector<int64_t>, LtGemm> cache;
    const std::vector<int64_t> key{dev, ta, tb, m, n, k, (int64_t)t, beta != 0.f};
    LtGemm &g = cache[key];
    if (!g.desc) {
        const hipblasOperation_t opa = ta ? HIPBLAS_OP_T : HIPBLAS_OP_N;
        const hipblasOperation_t opb = tb ? HIPBLAS_OP_T : HIPBLAS_OP_N;
        bool good = hipblasLtMatmulDescCreate(&g.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS;
        good = good && hipblasLtMatmulDescSetAttribute(g.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opa,
                                                       sizeof(opa)) == HIPBLAS_STATUS_SUCCESS;
        good = good && hipblasLtMatmulDescSetAttribute(g.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opb,
                                                       sizeof(opb)) == HIPBLAS_STATUS_SUCCESS;
        good = good && hipblasLtMatrixLayoutCreate(&g.a, t, ta ? k : m, ta ? m : k, ta ? k : m) == HIPBLAS_STATUS_SUCCESS;
        good = good && hipblasLtMatrixLayoutCreate(&g.b, t, tb ? n : k, tb ? k : n, tb ? n : k) ==
                           HIPBLAS_STATUS_SUCCESS;
        good = good && hipblasLtMatrixLayoutCreate(&g.c, HIP_R_32F, m, n, m) == HIPBLAS_STATUS_SUCCESS;
        hipblasLtMatmulPreference_t pref = nullptr;
        good = good && hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS;
        const uint64_t wsb = kLtWorkspace;
        good = good && hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                             &wsb, sizeof(wsb)) == HIPBLAS_STATUS_SUCCESS;
        hipblasLtMatmulHeuristicResult_t res[1];
        int found = 0;
        good = good && hipblasLtMatmulAlgoGetHeuristic(h, g.desc, g.a, g.b, g.c, g.c, pref, 1, res,
                                                       &found) == HIPBLAS_STATUS_SUCCESS;
        if (pref) hipblasLtMatmulPreferenceDestroy(pref);
        g.ok = good && found > 0 && res[0].workspaceSize <= kLtWorkspace;
        if (g.ok) g.algo = res[0].algo;
    }
    if (!g.ok) {
        set_error("hipBLASLt has no algorithm for a " + std::to_string(m) + " x " +
                  std::to_string(n) + " x " + std::to_string(k) + " product");
        return DM_ERR_HIP;
    }
    const float one = 1.f;
    const hipblasStatus_t s = hipblasLtMatmul(h, g.desc, &one, A, g.a, B, g.b, &beta, Dm, g.c, Dm,
                                              g.c, &g.algo, ws, kLtWorkspace, st);
    if (s != HIPBLAS_STATUS_SUCCESS) {
        set_error("hipBLASLt matmul failed (status " + std::to_string((int)s) + ")");
        return DM_ERR_HIP;
    }
    return DM_OK;
}

struct LpPlan {
    int64_t block, chunk;  // rows per block, vocabulary tokens per chunk
    bool bf16;             // both operands bf16 (else both taken as f32)
    size_t off_bits, off_state, off_z, off_e, off_h, off_w, off_lt, off_coef, off_gh, off_gw;
    size_t total;
};

// What a call holds: grad (the log-probability's softmax weights, two bf16 parts or f32),
// dz (the loss's logits gradient, bf16 or f32), and the loss's f32 gradient accumulators when
// the gradients' dtype is not f32.
static LpPlan lp_plan(const dm_logprob_desc *d, bool grad, bool dz, bool gh32, bool gw32) {
    LpPlan p{};
    const int64_t nb = d->n > 0 ? (d->n + d->row_chunk - 1) / d->row_chunk : 1;
    p.block = std::max<int64_t>(1, (d->n + nb - 1) / nb);
    // 0: 8192 tokens (measured best on MI355X for every block size); wider chunks are walked
    // 8192 tokens at a time (the statistics kernel holds a chunk's logits in registers)
    p.chunk = d->vocab_chunk > 0 ? d->vocab_chunk : kLpMaxChunk;
    p.chunk = std::min<int64_t>({p.chunk, kLpMaxChunk, std::max<int64_t>(d->v, 1)});
    p.bf16 = d->hidden_dtype == DM_BF16 && d->weight_dtype == DM_BF16;
    const int64_t n1 = std::max<int64_t>(d->n, 1);
    size_t o = 0;
    p.off_bits = o;
    o += align_up((size_t)((d->v + 31) / 32) * 4);
    p.off_state = o;
    o += align_up((size_t)LP_NSTATE * n1 * 4);
    p.off_z = o;
    o += align_up((size_t)p.block * p.chunk * 4);
    p.off_e = o;
    if (grad || dz) o += align_up((size_t)p.block * p.chunk * 4) + 256;
    p.off_h = o;
    if (!p.bf16 && d->hidden_dtype != DM_F32) o += align_up((size_t)d->n * d->d * 4);
    p.off_w = o;
    if (!p.bf16 && d->weight_dtype != DM_F32) o += align_up((size_t)d->v * d->d * 4);
    p.off_coef = o;
    if (dz) o += align_up((size_t)LC_COUNT * n1 * 4);
    p.off_gh = o;
    if (gh32) o += align_up((size_t)d->n * d->d * 4);
    p.off_gw = o;
    if (gw32) o += align_up((size_t)d->v * d->d * 4);
    p.off_lt = o;
    o += kLtWorkspace;
    p.total = o;
    return p;
}

static int lp_check(const std::string &op, const dm_logprob_desc *d, bool f16) {
    if (!d) return refuse(op + ": null descriptor");
    if (d->n < 0 || d->v < 1 || d->d < 1)
        return refuse(op + ": hidden is [n, D] and weight [V, D] with V, D >= 1");
    if (d->row_chunk < 1) return refuse(op + ": row_chunk must be at least 1");
    if (d->d % 8 != 0)
        return refuse(op + ": hidden widths D that are not a multiple of 8 are not implemented");
    if (d->vocab_chunk < 0) return refuse(op + ": vocab_chunk must not be negative");
    for (int dt : {d->hidden_dtype, d->weight_dtype})
        if (dt != DM_BF16 && dt != DM_F32 && !(f16 && dt == DM_F16))
            return refuse(op + (f16 ? ": the loss takes f32, bf16 or f16"
                                    : ": the log-probability takes bf16 or f32"));
    return DM_OK;
}

// The masked ids as words of bits, on the host (the ids are a host list, as the reference's
// Vec<u32>): each below V, at least one token left. Returns the number of distinct ids, or -1
// after a refusal.
static int64_t lp_bits(const std::string &op, const dm_logprob_desc *d, const uint32_t *masked,
                       int64_t n_masked, std::vector<uint32_t> &bits) {
    if (n_masked < 0 || (n_masked > 0 && !masked)) {
        refuse(op + ": masked ids need a host array of n_masked ids");
        return -1;
    }
    bits.assign((size_t)(d->v + 31) / 32, 0u);
    int64_t distinct = 0;
    for (int64_t i = 0; i < n_masked; i++) {
        const uint32_t id = masked[i];
        if ((int64_t)id >= d->v) {
            refuse(op + ": masked token id " + std::to_string(id) +
                   " is not below the vocabulary size " + std::to_string(d->v));
            return -1;
        }
        uint32_t &w = bits[id >> 5];
        if (!((w >> (id & 31)) & 1u)) distinct++;
        w |= 1u << (id & 31);
    }
    if (distinct >= d->v) {
        refuse(op + ": at least one token must stay unmasked");
        return -1;
    }
    return distinct;
}

// The operands in one arithmetic: both bf16, or both f32 (a bf16 or f16 one widened into the
// workspace).
static int lp_operands(const dm_logprob_desc *d, const LpPlan &p, const void *hidden,
                       const void *weight, char *ws, hipStream_t st, const void **H,
                       const void **W) {
    *H = hidden;
    *W = weight;
    if (p.bf16) return DM_OK;
    const void *src[2] = {hidden, weight};
    const int dts[2] = {d->hidden_dtype, d->weight_dtype};
    const int64_t counts[2] = {d->n * d->d, d->v * d->d};
    float *dst[2] = {(float *)(ws + p.off_h), (float *)(ws + p.off_w)};
    const void **out[2] = {H, W};
    for (int k = 0; k < 2; k++) {
        if (dts[k] == DM_F32) continue;
        if (dts[k] == DM_BF16)
            lp_widen<<<1024, 256, 0, st>>>(counts[k], (const uint16_t *)src[k], dst[k]);
        else
            lp_widen16<<<1024, 256, 0, st>>>(counts[k], (const _Float16 *)src[k], dst[k]);
        *out[k] = dst[k];
    }
    DM_LAUNCH_CHECK("widening the operands");
    return DM_OK;
}

// One block's logits of one chunk: Z (column-major cw x rows, i.e. [rows, cw] row-major) =
// W_c H_b^T; W_c is stored D x cw column-major, so op(A) = T.
static int lp_logits(const dm_logprob_desc *d, const LpPlan &p, const void *H, const void *W,
                     int64_t r0, int64_t rows, int64_t c0, int64_t cw, float *Z, void *lt_ws,
                     hipStream_t st) {
    const size_t esz = p.bf16 ? 2 : 4;
    return lt_gemm(st, true, false, cw, rows, d->d, (const char *)W + (size_t)c0 * d->d * esz,
                   (const char *)H + (size_t)r0 * d->d * esz, p.bf16 ? HIP_R_16BF : HIP_R_32F,
                   0.f, Z, lt_ws);
}

// The pass over the vocabulary (reference.rs:121-287): per block of rows and chunk, the logits
// and the statistics; with `grad`, o += E W_c in grad's rows. State [LP_NSTATE, n].
static int lp_pass(const dm_logprob_desc *d, const LpPlan &p, const void *H, const void *W,
                   const int64_t *targets, const uint32_t *dbits, char *ws, float *grad,
                   hipStream_t st, const std::function<int(int64_t, int64_t)> &after_block) {
    float *state = (float *)(ws + p.off_state);
    float *Z = (float *)(ws + p.off_z);
    void *E = ws + p.off_e;
    void *lt_ws = ws + p.off_lt;
    const hipDataType op_t = p.bf16 ? HIP_R_16BF : HIP_R_32F;
    const size_t esz = p.bf16 ? 2 : 4;
    const bool want_grad = grad != nullptr;
    for (int64_t r0 = 0; r0 < d->n; r0 += p.block) {
        const int64_t rows = std::min<int64_t>(p.block, d->n - r0);
        float *o = want_grad ? grad + r0 * d->d : nullptr;
        lp_init<<<(unsigned)rows, kLpThreads, 0, st>>>(rows, d->d, state + r0, d->n, o);
        DM_LAUNCH_CHECK("init");
        for (int64_t c0 = 0; c0 < d->v; c0 += p.chunk) {
            const int64_t cw = std::min<int64_t>(p.chunk, d->v - c0);
            // the bf16 remainder after the part, at an aligned offset
            void *E2 = (char *)E + align_up((size_t)rows * cw * 2);
            if (int rc = lp_logits(d, p, H, W, r0, rows, c0, cw, Z, lt_ws, st)) return rc;
            {
                KernelTimer timer(DM_KERNEL_LOGPROB_STATS, st);
                const int nv = (int)((cw + 1023) / 1024);
#define LP_STATS(EK, NV, EE, OO)                                                               \
    lp_stats<EK, NV><<<(unsigned)rows, kLpThreads, 0, st>>>(rows, cw, c0, d->d, Z, targets + r0, \
                                                            dbits, state + r0, d->n, EE, E2, OO)
#define LP_NV(EK, EE, OO)                          \
    if (nv <= 1) LP_STATS(EK, 1, EE, OO);          \
    else if (nv <= 2) LP_STATS(EK, 2, EE, OO);     \
    else if (nv <= 4) LP_STATS(EK, 4, EE, OO);     \
    else LP_STATS(EK, 8, EE, OO)
                if (!want_grad) {
                    LP_NV(0, nullptr, nullptr);
                } else if (p.bf16) {
                    LP_NV(1, E, o);
                } else {
                    LP_NV(2, E, o);
                }
#undef LP_NV
#undef LP_STATS
            }
            DM_LAUNCH_CHECK("statistics");
            if (want_grad) {
                // o (column-major D x rows) += W_c as stored (D x cw) E^T (cw x rows)
                const char *Wc = (const char *)W + (size_t)c0 * d->d * esz;
                for (int part = 0; part < (p.bf16 ? 2 : 1); part++)
                    if (int rc = lt_gemm(st, false, false, d->d, rows, cw, Wc, part ? E2 : E,
                                         op_t, 1.f, o, lt_ws))
                        return rc;
            }
        }
        if (int rc = after_block(r0, rows)) return rc;
    }
    return DM_OK;
}

static int lp_upload_bits(const std::vector<uint32_t> &bits, char *ws, const LpPlan &p,
                          hipStream_t st) {
    if (hipMemcpyAsync(ws + p.off_bits, bits.data(), bits.size() * 4, hipMemcpyHostToDevice, st) !=
        hipSuccess)
        return hip_status(hipGetLastError(), "copying the masked ids");
    return DM_OK;
}

static int lce_check(const dm_lce_desc *d) {
    const std::string op = "linear_cross_entropy";
    if (!d) return refuse(op + ": null descriptor");
    if (int rc = lp_check(op, &d->lp, true)) return rc;
    if (d->lp.hidden_dtype != d->lp.weight_dtype)
        return refuse(op + ": hidden and weight share one dtype");
    if (!(d->label_smoothing >= 0.f && d->label_smoothing <= 1.f))
        return refuse(op + ": label_smoothing must be in 0..=1, got " +
                      std::to_string(d->label_smoothing));
    if (!(std::isfinite(d->z_loss) && d->z_loss >= 0.f))
        return refuse(op + ": z_loss must be finite and at least 0, got " +
                      std::to_string(d->z_loss));
    return DM_OK;
}

}  // namespace dm

using namespace dm;

extern "C" {

size_t dm_chosen_logprob_workspace(const dm_logprob_desc *d, int with_grad) {
    if (lp_check("chosen_logprob", d, false) != DM_OK) return 0;
    return lp_plan(d, with_grad != 0, false, false, false).total;
}

int dm_chosen_logprob(const dm_logprob_desc *d, const void *hidden, const void *weight,
                      const int64_t *targets, const uint32_t *masked, int64_t n_masked,
                      float *logprob, float *entropy, float *grad, void *workspace,
                      size_t workspace_bytes, void *stream) {
    const std::string op = "chosen_logprob";
    if (int rc = lp_check(op, d, false)) return rc;
    std::vector<uint32_t> bits;
    if (lp_bits(op, d, masked, n_masked, bits) < 0) return DM_ERR_REFUSED;
    const bool want_grad = grad != nullptr;
    const LpPlan p = lp_plan(d, want_grad, false, false, false);
    if (workspace_bytes < p.total)
        return refuse(op + ": the workspace is smaller than dm_chosen_logprob_workspace");
    if (d->n == 0) return DM_OK;
    hipStream_t st = (hipStream_t)stream;
    char *ws = (char *)workspace;
    if (int rc = lp_upload_bits(bits, ws, p, st)) return rc;
    const void *H, *W;
    if (int rc = lp_operands(d, p, hidden, weight, ws, st, &H, &W)) return rc;
    const float *state = (const float *)(ws + p.off_state);
    int rc = lp_pass(d, p, H, W, targets, (const uint32_t *)(ws + p.off_bits), ws, grad, st,
                     [&](int64_t r0, int64_t rows) -> int {
                         float *o = want_grad ? grad + r0 * d->d : nullptr;
                         if (d->weight_dtype == DM_BF16)
                             lp_finish<DM_BF16><<<(unsigned)rows, kLpThreads, 0, st>>>(
                                 rows, d->v, d->d, state + r0, d->n, targets + r0, weight,
                                 logprob + r0, entropy + r0, o);
                         else
                             lp_finish<DM_F32><<<(unsigned)rows, kLpThreads, 0, st>>>(
                                 rows, d->v, d->d, state + r0, d->n, targets + r0, weight,
                                 logprob + r0, entropy + r0, o);
                         DM_LAUNCH_CHECK("chosen_logprob: finish");
                         return DM_OK;
                     });
    if (rc) return rc;
    probe_add(DM_PROBE_LOGPROB);
    return DM_OK;
}

size_t dm_linear_cross_entropy_workspace(const dm_lce_desc *d, int backward) {
    if (lce_check(d) != DM_OK) return 0;
    const bool f32 = d->lp.hidden_dtype == DM_F32;
    // backward 1: both gradients; 2: the hidden's alone (no weight-gradient accumulator)
    return lp_plan(&d->lp, false, backward != 0, backward && !f32, backward == 1 && !f32).total;
}

int dm_linear_cross_entropy_fwd(const dm_lce_desc *d, const void *hidden, const void *weight,
                                const int64_t *targets, const uint32_t *masked, int64_t n_masked,
                                float *rows, void *workspace, size_t workspace_bytes,
                                void *stream) {
    const std::string op = "linear_cross_entropy";
    if (int rc = lce_check(d)) return rc;
    const dm_logprob_desc *lp = &d->lp;
    std::vector<uint32_t> bits;
    const int64_t nmask = lp_bits(op, lp, masked, n_masked, bits);
    if (nmask < 0) return DM_ERR_REFUSED;
    const LpPlan p = lp_plan(lp, false, false, false, false);
    if (workspace_bytes < p.total)
        return refuse(op + ": the workspace is smaller than dm_linear_cross_entropy_workspace");
    if (lp->n == 0) return DM_OK;
    hipStream_t st = (hipStream_t)stream;
    char *ws = (char *)workspace;
    if (int rc = lp_upload_bits(bits, ws, p, st)) return rc;
    const void *H, *W;
    if (int rc = lp_operands(lp, p, hidden, weight, ws, st, &H, &W)) return rc;
    if (int rc = lp_pass(lp, p, H, W, targets, (const uint32_t *)(ws + p.off_bits), ws, nullptr,
                         st, [](int64_t, int64_t) { return (int)DM_OK; }))
        return rc;
    const float inv_classes = 1.f / (float)(lp->v - nmask);
    lce_finish<<<(unsigned)((lp->n + 255) / 256), 256, 0, st>>>(
        lp->n, (const float *)(ws + p.off_state), targets, d->ignore_index, d->label_smoothing,
        d->z_loss, inv_classes, rows);
    DM_LAUNCH_CHECK("linear_cross_entropy: finish");
    probe_add(DM_PROBE_LCE_FWD);
    return DM_OK;
}

int dm_linear_cross_entropy_bwd(const dm_lce_desc *d, const void *hidden, const void *weight,
                                const int64_t *targets, const uint32_t *masked, int64_t n_masked,
                                const float *rows, const float *upstream, void *grad_hidden,
                                void *grad_weight, void *workspace, size_t workspace_bytes,
                                void *stream) {
    const std::string op = "linear_cross_entropy";
    if (int rc = lce_check(d)) return rc;
    const dm_logprob_desc *lp = &d->lp;
    std::vector<uint32_t> bits;
    const int64_t nmask = lp_bits(op, lp, masked, n_masked, bits);
    if (nmask < 0) return DM_ERR_REFUSED;
    const bool f32 = lp->hidden_dtype == DM_F32;
    // the weight-gradient accumulator (16-bit inputs) is reserved only when that gradient is
    // asked for: dm_linear_cross_entropy_workspace(desc, 2) sizes a call without it
    const LpPlan p = lp_plan(lp, false, true, !f32, !f32 && grad_weight != nullptr);
    if (workspace_bytes < p.total)
        return refuse(op + ": the workspace is smaller than dm_linear_cross_entropy_workspace");
    hipStream_t st = (hipStream_t)stream;
    char *ws = (char *)workspace;
    float *gh = grad_hidden ? (f32 ? (float *)grad_hidden : (float *)(ws + p.off_gh)) : nullptr;
    float *gw = grad_weight ? (f32 ? (float *)grad_weight : (float *)(ws + p.off_gw)) : nullptr;
    // (the accumulators need no clearing: the first row block's products write grad_weight and
    // each row block's first chunk writes its rows of grad_hidden, with beta = 0)
    if (lp->n == 0) {
        if (gw) {
            lp_zero<<<1024, 256, 0, st>>>(lp->v * lp->d, gw);
            DM_LAUNCH_CHECK("linear_cross_entropy: zero");
        }
        if (grad_weight && !f32) {
            lp_cast<<<1024, 256, 0, st>>>(lp->v * lp->d, gw, grad_weight, lp->weight_dtype);
            DM_LAUNCH_CHECK("linear_cross_entropy: cast");
        }
        return DM_OK;
    }
    if (int rc = lp_upload_bits(bits, ws, p, st)) return rc;
    const void *H, *W;
    if (int rc = lp_operands(lp, p, hidden, weight, ws, st, &H, &W)) return rc;
    const float inv_classes = 1.f / (float)(lp->v - nmask);
    float *coef = (float *)(ws + p.off_coef);
    lce_coef<<<(unsigned)((lp->n + 255) / 256), 256, 0, st>>>(
        lp->n, rows, upstream, d->label_smoothing, d->z_loss, inv_classes, d->entropy, coef);
    DM_LAUNCH_CHECK("linear_cross_entropy: coefficients");
    // the gradient pass (logprob/reference.rs:289-380): the logits again, the logits' gradient,
    // then grad_hidden_b += G W_c and grad_weight_c += G^T H_b
    float *Z = (float *)(ws + p.off_z);
    void *G = ws + p.off_e, *lt_ws = ws + p.off_lt;
    const hipDataType op_t = p.bf16 ? HIP_R_16BF : HIP_R_32F;
    const size_t esz = p.bf16 ? 2 : 4;
    const uint32_t *dbits = (const uint32_t *)(ws + p.off_bits);
    for (int64_t r0 = 0; r0 < lp->n; r0 += p.block) {
        const int64_t rows_b = std::min<int64_t>(p.block, lp->n - r0);
        for (int64_t c0 = 0; c0 < lp->v; c0 += p.chunk) {
            const int64_t cw = std::min<int64_t>(p.chunk, lp->v - c0);
            if (int rc = lp_logits(lp, p, H, W, r0, rows_b, c0, cw, Z, lt_ws, st)) return rc;
            if (p.bf16)
                lce_dz<true><<<(unsigned)rows_b, kLpThreads, 0, st>>>(
                    rows_b, cw, c0, Z, targets + r0, dbits, rows + r0, coef + r0, lp->n, G);
            else
                lce_dz<false><<<(unsigned)rows_b, kLpThreads, 0, st>>>(
                    rows_b, cw, c0, Z, targets + r0, dbits, rows + r0, coef + r0, lp->n, G);
            DM_LAUNCH_CHECK("linear_cross_entropy: logits gradient");
            const char *Wc = (const char *)W + (size_t)c0 * lp->d * esz;
            // grad_hidden (column-major D x rows) += W_c as stored (D x cw) G^T (cw x rows).
            // The first product of each accumulator runs with beta = 0, which hipBLASLt takes
            // as "C is not read" (the accumulators are never cleared; a workspace poisoned with
            // NaN gives the same bits as a zeroed one, a property the GPU tests hold it to)
            if (gh)
                if (int rc = lt_gemm(st, false, false, lp->d, rows_b, cw, Wc, G, op_t,
                                     c0 == 0 ? 0.f : 1.f, gh + r0 * lp->d, lt_ws))
                    return rc;
            // grad_weight_c (column-major D x cw) += H_b as stored (D x rows) G (rows x cw; G
            // is stored cw x rows, so op(B) = T)
            if (gw)
                if (int rc = lt_gemm(st, false, true, lp->d, cw, rows_b,
                                     (const char *)H + (size_t)r0 * lp->d * esz, G, op_t,
                                     r0 == 0 ? 0.f : 1.f, gw + c0 * lp->d, lt_ws))
                    return rc;
        }
    }
    if (!f32) {
        if (grad_hidden) lp_cast<<<1024, 256, 0, st>>>(lp->n * lp->d, gh, grad_hidden, lp->hidden_dtype);
        if (grad_weight) lp_cast<<<1024, 256, 0, st>>>(lp->v * lp->d, gw, grad_weight, lp->weight_dtype);
        DM_LAUNCH_CHECK("linear_cross_entropy: cast");
    }
    probe_add(DM_PROBE_LCE_BWD);
    return DM_OK;
}

}  // extern "C"
