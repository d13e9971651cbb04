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

#include <cfloat>
#include <algorithm>
#include <map>
#include <string>
#include <vector>

#include "attention_kernels.h"
#include "dm_common.h"

namespace dm {

enum { LP_M = 0, LP_S, LP_R, LP_A, LP_ZT, LP_FOUND, LP_NSTATE };

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
    const float m = st[LP_M * nst + row];
    const float m_new = mx > m ? mx : m;
    const float shift = m - m_new, alpha = expf(shift);
    const int64_t t = targets[row];
    const int64_t tl = t - c0;
    const bool has_t = tl >= 0 && tl < cw && !lp_masked(bits, t);
    // the chunk's sums; the weights of the next product (0 for the target and masked tokens)
    float se = 0.f, sa = 0.f, sr = 0.f;
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
    sa = lp_block_sum(sa, sm);
    sr = lp_block_sum(sr, sm);
    if constexpr (EK != 0) {
        // o is still zero while nothing has been summed (the first chunk)
        if (alpha != 1.f && st[LP_S * nst + row] != 0.f)
            for (int64_t e = threadIdx.x; e < D; e += kLpThreads) o[row * D + e] *= alpha;
    }
    if (threadIdx.x == 0) {
        const float s = st[LP_S * nst + row], a = st[LP_A * nst + row];
        st[LP_A * nst + row] = alpha * (a + s * shift) + sa;
        st[LP_S * nst + row] = s * alpha + se;
        st[LP_R * nst + row] = st[LP_R * nst + row] * alpha + sr;
        if (has_t) {
            st[LP_ZT * nst + row] += z[tl];
            st[LP_FOUND * nst + row] += 1.f;
        }
        st[LP_M * nst + row] = m_new;
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
// type `t`, A stored m x k (ta = N, lda m) or k x m (ta = T, lda k), B k x n (ld k).
static int lt_gemm(hipStream_t st, bool ta, int64_t m, int64_t n, int64_t k, const void *A,
                   const void *B, hipDataType t, float beta, float *Dm, void *ws) {
    hipblasLtHandle_t h = lt_handle();
    if (!h) {
        set_error("chosen_logprob: no hipBLASLt handle");
        return DM_ERR_HIP;
    }
    int dev = 0;
    (void)hipGetDevice(&dev);
    thread_local std::map<std::vector<int64_t>, LtGemm> cache;
    const std::vector<int64_t> key{dev, ta, m, n, k, (int64_t)t, beta != 0.f};
    LtGemm &g = cache[key];
    if (!g.desc) {
        const hipblasOperation_t opa = ta ? HIPBLAS_OP_T : HIPBLAS_OP_N, opb = HIPBLAS_OP_N;
        bool good = hipblasLtMatmulDescCreate(&g.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS;
        good = good && hipblasLtMatmulDescSetAttribute(g.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opa,
                                                       sizeof(opa)) == HIPBLAS_STATUS_SUCCESS;
        good = good && hipblasLtMatmulDescSetAttribute(g.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opb,
                                                       sizeof(opb)) == HIPBLAS_STATUS_SUCCESS;
        good = good && hipblasLtMatrixLayoutCreate(&g.a, t, ta ? k : m, ta ? m : k, ta ? k : m) == HIPBLAS_STATUS_SUCCESS;
        good = good && hipblasLtMatrixLayoutCreate(&g.b, t, k, n, k) == HIPBLAS_STATUS_SUCCESS;
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
        set_error("chosen_logprob: hipBLASLt has no algorithm for a " + std::to_string(m) + " x " +
                  std::to_string(n) + " x " + std::to_string(k) + " product");
        return DM_ERR_HIP;
    }
    const float one = 1.f;
    const hipblasStatus_t s = hipblasLtMatmul(h, g.desc, &one, A, g.a, B, g.b, &beta, Dm, g.c, Dm,
                                              g.c, &g.algo, ws, kLtWorkspace, st);
    if (s != HIPBLAS_STATUS_SUCCESS) {
        set_error("chosen_logprob: hipBLASLt matmul failed (status " + std::to_string((int)s) + ")");
        return DM_ERR_HIP;
    }
    return DM_OK;
}

struct LpPlan {
    int64_t block, chunk;  // rows per block, vocabulary tokens per chunk
    bool bf16;             // both operands bf16 (else both taken as f32)
    size_t off_bits, off_state, off_z, off_e, off_h, off_w, off_lt, total;
};

static LpPlan lp_plan(const dm_logprob_desc *d, bool grad) {
    LpPlan p{};
    const int64_t nb = d->n > 0 ? (d->n + d->row_chunk - 1) / d->row_chunk : 1;
    p.block = std::max<int64_t>(1, (d->n + nb - 1) / nb);
    // 0: 8192 tokens (measured best on MI355X for every block size); wider chunks are walked
    // 8192 tokens at a time (the statistics kernel holds a chunk's logits in registers)
    p.chunk = d->vocab_chunk > 0 ? d->vocab_chunk : kLpMaxChunk;
    p.chunk = std::min<int64_t>({p.chunk, kLpMaxChunk, std::max<int64_t>(d->v, 1)});
    p.bf16 = d->hidden_dtype == DM_BF16 && d->weight_dtype == DM_BF16;
    size_t o = 0;
    p.off_bits = o;
    o += align_up((size_t)((d->v + 31) / 32) * 4);
    p.off_state = o;
    o += align_up((size_t)LP_NSTATE * std::max<int64_t>(d->n, 1) * 4);
    p.off_z = o;
    o += align_up((size_t)p.block * p.chunk * 4);
    p.off_e = o;
    if (grad) o += align_up((size_t)p.block * p.chunk * 4) + 256;  // two bf16 parts or one f32
    p.off_h = o;
    if (!p.bf16 && d->hidden_dtype == DM_BF16) o += align_up((size_t)d->n * d->d * 4);
    p.off_w = o;
    if (!p.bf16 && d->weight_dtype == DM_BF16) o += align_up((size_t)d->v * d->d * 4);
    p.off_lt = o;
    o += kLtWorkspace;
    p.total = o;
    return p;
}

static int lp_check(const dm_logprob_desc *d) {
    if (!d) return refuse("chosen_logprob: null descriptor");
    if (d->n < 0 || d->v < 1 || d->d < 1)
        return refuse("chosen_logprob: hidden is [n, D] and weight [V, D] with V, D >= 1");
    if (d->row_chunk < 1) return refuse("chosen_logprob: row_chunk must be at least 1");
    if (d->d % 8 != 0)
        return refuse("chosen_logprob: hidden widths D that are not a multiple of 8 are not "
                      "implemented");
    if (d->vocab_chunk < 0) return refuse("chosen_logprob: vocab_chunk must not be negative");
    for (int dt : {d->hidden_dtype, d->weight_dtype})
        if (dt != DM_BF16 && dt != DM_F32)
            return refuse("chosen_logprob: the log-probability takes bf16 or f32");
    return DM_OK;
}


}  // namespace dm

using namespace dm;

extern "C" {

size_t dm_chosen_logprob_workspace(const dm_logprob_desc *d, int with_grad) {
    if (lp_check(d) != DM_OK) return 0;
    return lp_plan(d, with_grad != 0).total;
}

int dm_chosen_logprob(const dm_logprob_desc *d, const void *hidden, const void *weight,
                      const int64_t *targets, const uint32_t *masked, int64_t n_masked,
                      float *logprob, float *entropy, float *grad, void *workspace,
                      size_t workspace_bytes, void *stream) {
    if (int rc = lp_check(d)) return rc;
    if (n_masked < 0 || (n_masked > 0 && !masked))
        return refuse("chosen_logprob: masked ids need a host array of n_masked ids");
    // the masked ids as words of bits, on the host (the ids are a host list, as the
    // reference's Vec<u32>): each below V, at least one token left
    std::vector<uint32_t> bits((size_t)(d->v + 31) / 32, 0u);
    int64_t distinct = 0;
    for (int64_t i = 0; i < n_masked; i++) {
        const uint32_t id = masked[i];
        if ((int64_t)id >= d->v)
            return refuse("chosen_logprob: masked token id " + std::to_string(id) +
                          " is not below the vocabulary size " + std::to_string(d->v));
        uint32_t &w = bits[id >> 5];
        if (!((w >> (id & 31)) & 1u)) distinct++;
        w |= 1u << (id & 31);
    }
    if (distinct >= d->v) return refuse("chosen_logprob: at least one token must stay unmasked");
    const bool want_grad = grad != nullptr;
    const LpPlan p = lp_plan(d, want_grad);
    if (workspace_bytes < p.total)
        return refuse("chosen_logprob: the workspace is smaller than dm_chosen_logprob_workspace");
    if (d->n == 0) return DM_OK;
    hipStream_t st = (hipStream_t)stream;
    char *ws = (char *)workspace;
    uint32_t *dbits = (uint32_t *)(ws + p.off_bits);
    float *state = (float *)(ws + p.off_state);
    float *Z = (float *)(ws + p.off_z);
    void *E = ws + p.off_e;
    if (hipMemcpyAsync(dbits, bits.data(), bits.size() * 4, hipMemcpyHostToDevice, st) !=
        hipSuccess)
        return hip_status(hipGetLastError(), "chosen_logprob: copying the masked ids");

    // operands in one arithmetic: both bf16, or both f32 (a bf16 one widened)
    const void *H = hidden, *W = weight;
    if (!p.bf16) {
        if (d->hidden_dtype == DM_BF16) {
            lp_widen<<<1024, 256, 0, st>>>(d->n * d->d, (const uint16_t *)hidden,
                                           (float *)(ws + p.off_h));
            H = ws + p.off_h;
        }
        if (d->weight_dtype == DM_BF16) {
            lp_widen<<<1024, 256, 0, st>>>(d->v * d->d, (const uint16_t *)weight,
                                           (float *)(ws + p.off_w));
            W = ws + p.off_w;
        }
        DM_LAUNCH_CHECK("chosen_logprob: widen");
    }
    const hipDataType op_t = p.bf16 ? HIP_R_16BF : HIP_R_32F;
    const size_t esz = p.bf16 ? 2 : 4;
    void *lt_ws = ws + p.off_lt;
    for (int64_t r0 = 0; r0 < d->n; r0 += p.block) {
        const int64_t rows = std::min<int64_t>(p.block, d->n - r0);
        float *o = want_grad ? grad + r0 * d->d : nullptr;
        lp_init<<<(unsigned)rows, kLpThreads, 0, st>>>(rows, d->d, state + r0, d->n, o);
        DM_LAUNCH_CHECK("chosen_logprob: init");
        const char *Hb = (const char *)H + (size_t)r0 * d->d * esz;
        for (int64_t c0 = 0; c0 < d->v; c0 += p.chunk) {
            const int64_t cw = std::min<int64_t>(p.chunk, d->v - c0);
            // the bf16 remainder after the part, at an aligned offset
            void *E2 = (char *)E + align_up((size_t)rows * cw * 2);
            const char *Wc = (const char *)W + (size_t)c0 * d->d * esz;
            // Z (column-major cw x rows, i.e. [rows, cw] row-major) = W_c H^T: W_c is stored
            // D x cw column-major, so op(A) = T
            if (int rc = lt_gemm(st, true, cw, rows, d->d, Wc, Hb, op_t, 0.f, Z, lt_ws)) return rc;
            {
                KernelTimer timer(DM_KERNEL_LOGPROB_STATS, st);
                const int nv = (int)((cw + 1023) / 1024);
#define LP_STATS(EK, NV, EE, OO)                                                                   lp_stats<EK, NV><<<(unsigned)rows, kLpThreads, 0, st>>>(rows, cw, c0, d->d, Z, targets + r0,                                                             dbits, state + r0, d->n, EE, E2, OO)
#define LP_NV(EK, EE, OO)                                                                          if (nv <= 1) LP_STATS(EK, 1, EE, OO);                                                          else if (nv <= 2) LP_STATS(EK, 2, EE, OO);                                                     else if (nv <= 4) LP_STATS(EK, 4, EE, OO);                                                     else LP_STATS(EK, 8, EE, OO)
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
            DM_LAUNCH_CHECK("chosen_logprob: stats");
            if (want_grad) {
                // o (column-major D x rows) += W_c as stored (D x cw) E^T (cw x rows)
                const int parts = p.bf16 ? 2 : 1;
                for (int part = 0; part < parts; part++) {
                    const void *Ep = part ? E2 : E;
                    if (int rc = lt_gemm(st, false, d->d, rows, cw, Wc, Ep, op_t, 1.f, o, lt_ws))
                        return rc;
                }
            }
        }
        if (p.bf16 || d->weight_dtype == DM_BF16)
            lp_finish<DM_BF16><<<(unsigned)rows, kLpThreads, 0, st>>>(
                rows, d->v, d->d, state + r0, d->n, targets + r0, weight, logprob + r0,
                entropy + r0, o);
        else
            lp_finish<DM_F32><<<(unsigned)rows, kLpThreads, 0, st>>>(
                rows, d->v, d->d, state + r0, d->n, targets + r0, weight, logprob + r0,
                entropy + r0, o);
        DM_LAUNCH_CHECK("chosen_logprob: finish");
    }
    probe_add(DM_PROBE_LOGPROB);
    return DM_OK;
}

}  // extern "C"
