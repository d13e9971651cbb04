// The gated delta rule's recurrent step (crates/dash-ops/src/gated_delta/recurrent.rs:158,
// recurrent/kernel.rs:36-408): one workgroup per (sequence, head) holds the [Dk, Dv] f32 state
// in registers for all of the sequence's tokens of the call, so the state is read from HBM once
// and written once; bandwidth-bound, no MFMA.
//
// Thread layout: the state's columns in groups of 4 (float4 loads and stores along Dv, a
// wavefront covering whole 64-column rows), and the rows split among NKG row groups; the two
// reductions over Dk of each token (S^T k and S^T q) go through LDS.
#include <string>

#include "attention_kernels.h"
#include "gdr_common.h"

namespace dm {

// Per token, with S the state (recurrent.rs:362-396):
//   q, k <- l2norm (optional), q <- scale q;  S <- exp(g) S;  delta <- beta (v - S^T k);
//   S <- S + k delta^T;  out <- S^T q.
template <int DT, int MAXR>
__global__ __launch_bounds__(256) void gdr_step_kernel(
    GdrArgs a, int64_t nseq, int64_t Dk, int64_t Dv, int ncs, const int32_t *__restrict__ cu,
    const float *state_in, float *state_out, void *__restrict__ out) {
    const int64_t H = a.H;
    const int g_dt = a.g_dt, beta_dt = a.beta_dt, l2norm = a.l2norm;
    const float scale = a.scale;
    const void *q = a.q, *k = a.k, *v = a.v, *g = a.g, *beta = a.beta;
    // the state's columns are independent: ncs workgroups share a (sequence, head), each
    // taking Dv / ncs columns (every one recomputes the token's normalisation)
    const int64_t sh = blockIdx.x / ncs;
    const int64_t s = sh / H, h = sh % H;
    const int64_t Dw = Dv / ncs, c0 = (blockIdx.x % ncs) * Dw;
    const int tid = threadIdx.x;
    const int NQ = (int)(Dw / 4);       // column quads
    const int NKG = 256 / NQ;           // row groups
    const int quad = tid % NQ, kg = tid / NQ;
    const bool active = kg < NKG;
    const int rows_per = (int)((Dk + NKG - 1) / NKG);
    const int r0 = kg * rows_per;

    extern __shared__ float sm[];
    float *qs = sm;            // [Dk]
    float *ks = qs + Dk;       // [Dk]
    float *red = ks + Dk;      // [NKG][Dw] partial sums
    __shared__ float norm2[2];

    int64_t t0, t1;
    if (cu) {
        t0 = cu[s];
        t1 = cu[s + 1];
    } else {
        t0 = s;
        t1 = s + 1;
    }

    float st_[MAXR][4];
    const float *sin = state_in + sh * Dk * Dv;
#pragma unroll
    for (int rr = 0; rr < MAXR; rr++) {
        const int64_t row = r0 + rr;
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
        if (active && rr < rows_per && row < Dk) x = *(const float4 *)(sin + row * Dv + c0 + quad * 4);
        st_[rr][0] = x.x;
        st_[rr][1] = x.y;
        st_[rr][2] = x.z;
        st_[rr][3] = x.w;
    }

    for (int64_t t = t0; t < t1; t++) {
        const int64_t q_off = q_at(a, t, h), k_off = k_at(a, t, h);
        // load q, k (f32), normalise
        float pq = 0.f, pk = 0.f;
        for (int64_t x = tid; x < Dk; x += 256) {
            const float qv = ld<DT>(q, q_off + x), kv = ld<DT>(k, k_off + x);
            qs[x] = qv;
            ks[x] = kv;
            pq += qv * qv;
            pk += kv * kv;
        }
        if (l2norm) {
            pq = wave_sum(pq);
            pk = wave_sum(pk);
            if (tid == 0) norm2[0] = norm2[1] = 0.f;
            __syncthreads();
            if ((tid & 63) == 0) {
                atomicAdd(&norm2[0], pq);
                atomicAdd(&norm2[1], pk);
            }
        }
        __syncthreads();
        float qmul = scale, kmul = 1.f;
        if (l2norm) {
            // x * (1 / sqrt(sum x^2 + eps)) (recurrent.rs:400-404)
            qmul = (1.f / sqrtf(norm2[0] + 1e-6f));
            kmul = 1.f / sqrtf(norm2[1] + 1e-6f);
        }
        const float decay = expf(ld_any(g_dt, g, g_at(a, t, h)));
        const float bt = ld_any(beta_dt, beta, b_at(a, t, h));

        // S <- exp(g) S ; partial S^T k
        float part[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int rr = 0; rr < MAXR; rr++) {
            const int64_t row = r0 + rr;
            const float kr = (active && rr < rows_per && row < Dk) ? ks[row] * kmul : 0.f;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                st_[rr][c] *= decay;
                part[c] += st_[rr][c] * kr;
            }
        }
        if (active)
#pragma unroll
            for (int c = 0; c < 4; c++) red[kg * Dw + quad * 4 + c] = part[c];
        __syncthreads();
        float delta[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            float kv = 0.f;
            for (int x = 0; x < NKG; x++) kv += red[x * Dw + quad * 4 + c];
            delta[c] = (ld<DT>(v, v_at(a, t, h) + c0 + quad * 4 + c) - kv) * bt;
        }
        __syncthreads();
        // S <- S + k delta^T ; partial S^T q
#pragma unroll
        for (int c = 0; c < 4; c++) part[c] = 0.f;
#pragma unroll
        for (int rr = 0; rr < MAXR; rr++) {
            const int64_t row = r0 + rr;
            const bool ok = active && rr < rows_per && row < Dk;
            const float kr = ok ? ks[row] * kmul : 0.f;
            const float qr = ok ? qs[row] * qmul * (l2norm ? scale : 1.f) : 0.f;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                st_[rr][c] += kr * delta[c];
                part[c] += st_[rr][c] * qr;
            }
        }
        if (active)
#pragma unroll
            for (int c = 0; c < 4; c++) red[kg * Dw + quad * 4 + c] = part[c];
        __syncthreads();
        if (kg == 0) {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                float o = 0.f;
                for (int x = 0; x < NKG; x++) o += red[x * Dw + quad * 4 + c];
                st<DT>(out, (t * H + h) * Dv + c0 + quad * 4 + c, o);
            }
        }
        __syncthreads();
    }

    float *sout = state_out + sh * Dk * Dv;
#pragma unroll
    for (int rr = 0; rr < MAXR; rr++) {
        const int64_t row = r0 + rr;
        if (active && rr < rows_per && row < Dk)
            *(float4 *)(sout + row * Dv + c0 + quad * 4) =
                make_float4(st_[rr][0], st_[rr][1], st_[rr][2], st_[rr][3]);
    }
}

int check_gdr(const dm_gdr_desc *d, const char *op, bool step) {
    std::string o(op);
    if (!d) return refuse(o + ": null descriptor");
    if (d->b < 0 || d->t < 0 || d->h < 0 || d->dk < 0 || d->dv < 0)
        return refuse(o + ": negative dimension");
    if (d->dtype != DM_F32 && d->dtype != DM_BF16 && d->dtype != DM_F16)
        return refuse(o + ": q, k and v must share one float dtype (f32, bf16 or f16)");
    if (d->g_dtype != DM_F32 && d->g_dtype != d->dtype)
        return refuse(o + ": g must be f32 or the inputs' dtype");
    if (d->beta_dtype != DM_F32 && d->beta_dtype != d->dtype)
        return refuse(o + ": beta must be f32 or the inputs' dtype");
    if (d->cu_seqlens) {
        if (d->nseq < 1) return refuse(o + ": cu_seqlens must hold S + 1 >= 2 offsets");
        if (!step && d->b != 1)
            return refuse(o + ": packed sequences lie along the time, B = 1");
    }
    if (d->dk > 256 || d->dv > 256)
        return refuse(o + ": heads wider than 256 are not implemented");
    if (!gdr_strides_ok(d, step))
        return refuse(o + ": strides must not be negative, and each batch stride must be T times "
                          "its time stride (the host copies other views)");
    return DM_OK;
}

}  // namespace dm

using namespace dm;

extern "C" int dm_gdr_step(const dm_gdr_desc *d, const void *q, const void *k, const void *v,
                           const void *g, const void *beta, const float *state_in,
                           float *state_out, void *out, void *stream) {
    int rc = check_gdr(d, "gated_delta_step", true);
    if (rc) return rc;
    if (d->dv % 4 != 0)
        return refuse("gated_delta_step: Dv must be a multiple of 4 (" + std::to_string(d->dv) +
                      ")");
    hipStream_t st = (hipStream_t)stream;
    const int64_t nseq = d->cu_seqlens ? d->nseq : d->b;
    // columns per workgroup: 64 where Dv allows it (more, shorter workgroups let the state's
    // reads and writes of different workgroups overlap)
    const int ncs = (d->dv >= 128 && d->dv % 64 == 0) ? (int)(d->dv / 64) : 1;
    const int64_t blocks = nseq * d->h * ncs;
    if (blocks == 0 || d->dk * d->dv == 0) return DM_OK;
    const int64_t dw = d->dv / ncs;
    const int nq = (int)(dw / 4);
    const int nkg = 256 / nq;
    const int rows = (int)((d->dk + nkg - 1) / nkg);
    const size_t smem = (size_t)(2 * d->dk + nkg * dw) * sizeof(float);
    const GdrArgs a = gdr_args(d, q, k, v, g, beta, true);
#define STEP(DT, R)                                                                          \
    gdr_step_kernel<DT, R><<<(unsigned)blocks, 256, smem, st>>>(                             \
        a, nseq, d->dk, d->dv, ncs, d->cu_seqlens, state_in, state_out, out)
#define STEP_R(DT)                                  \
    if (rows <= 4) STEP(DT, 4);                     \
    else if (rows <= 8) STEP(DT, 8);                \
    else if (rows <= 16) STEP(DT, 16);              \
    else if (rows <= 32) STEP(DT, 32);              \
    else STEP(DT, 64);
    if (rows > 64) return refuse("gated_delta_step: state shape not implemented");
    {
        KernelTimer timer(DM_KERNEL_GDR_STEP, st);
        if (d->dtype == DM_F32) {
            STEP_R(DM_F32)
        } else if (d->dtype == DM_BF16) {
            STEP_R(DM_BF16)
        } else {
            STEP_R(DM_F16)
        }
    }
#undef STEP_R
#undef STEP
    probe_add(DM_PROBE_GDR_STEP);
    DM_LAUNCH_CHECK("gated_delta_step: launch");
    return DM_OK;
}
