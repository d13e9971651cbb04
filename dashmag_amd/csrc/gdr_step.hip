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

// The columns a thread holds: 4 from column 4 * quad of its workgroup's slice; with VEC, one
// 16-byte access (the slice's width a multiple of 4 and the rows 16-byte aligned), otherwise
// element by element, those past the slice's width held at zero.
template <bool VEC>
__device__ __forceinline__ void ld_cols(const float *row, int cq, int64_t dw, float x[4]) {
    if (VEC) {
        float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
        if (cq < dw) y = *(const float4 *)(row + cq);
        x[0] = y.x, x[1] = y.y, x[2] = y.z, x[3] = y.w;
    } else {
#pragma unroll
        for (int c = 0; c < 4; c++) x[c] = cq + c < dw ? row[cq + c] : 0.f;
    }
}
template <bool VEC>
__device__ __forceinline__ void st_cols(float *row, int cq, int64_t dw, const float x[4]) {
    if (VEC) {
        if (cq < dw) *(float4 *)(row + cq) = make_float4(x[0], x[1], x[2], x[3]);
    } else {
#pragma unroll
        for (int c = 0; c < 4; c++)
            if (cq + c < dw) row[cq + c] = x[c];
    }
}

// Per token, with S the state (recurrent.rs:362-396):
//   q, k <- l2norm (optional), q <- scale q;  S <- exp(g) S;  delta <- beta (v - S^T k);
//   S <- S + k delta^T;  out <- S^T q.
// ONE: one token per sequence (no offsets), Dk = 128 and 64-column slices, every index and
// bound known at compile time.
template <int DT, bool VEC, int MAXR, bool ONE>
__global__ __launch_bounds__(256) void gdr_step_kernel(
    GdrArgs a, int64_t nseq, int64_t Dk_, int64_t Dv, int ncs, const int32_t *__restrict__ cu,
    const float *state_in, float *state_out, void *__restrict__ out) {
    static_assert(!ONE || (VEC && MAXR == 8), "the one-token form is the 8-row vector one");
    const int64_t Dk = ONE ? 128 : Dk_;
    const int64_t H = a.H;
    const int g_dt = a.g_dt, beta_dt = a.beta_dt, l2norm = a.l2norm;
    const float scale = a.scale;
    const void *q = a.q, *k = a.k, *v = a.v, *g = a.g, *beta = a.beta;
    // the state's columns are independent: ncs workgroups share a (sequence, head), each
    // taking Dv / ncs columns (every one recomputes the token's normalisation)
    const int64_t sh = blockIdx.x / ncs;
    const int64_t s = sh / H, h = sh % H;
    const int64_t Dw = ONE ? 64 : Dv / ncs, c0 = (blockIdx.x % ncs) * Dw;
    const int tid = threadIdx.x;
    const int NQ = (int)((Dw + 3) / 4);  // column quads
    const int NKG = 256 / NQ;            // row groups
    const int quad = tid % NQ, kg = tid / NQ;
    const int cq = quad * 4;
    const bool active = ONE || kg < NKG;
    const int rows_per = (int)((Dk + NKG - 1) / NKG);
    const int r0 = kg * rows_per;

    extern __shared__ float sm[];
    float *qs = sm;            // [Dk]
    float *ks = qs + Dk;       // [Dk]
    float *red = ks + Dk;      // [NKG][4 NQ] partial sums
    __shared__ float norm2[2][4];  // the wavefronts' sums of q^2 and k^2

    int64_t t0, t1;
    if (!ONE && cu) {
        t0 = cu[s];
        t1 = cu[s + 1];
    } else {
        t0 = s;
        t1 = s + 1;
    }

    float st_[MAXR][4];
    const float *sin = state_in + sh * Dk * Dv + c0;
    // a row's offset from the slice's first, in 32 bits (Dk x Dv is at most 2^16; 64-bit
    // products per row had doubled the registers of the one-token form)
    const int dv32 = (int)Dv;
#pragma unroll
    for (int rr = 0; rr < MAXR; rr++) {
        const int64_t row = r0 + rr;
        if (ONE || (active && rr < rows_per && row < Dk))
            ld_cols<VEC>(sin + r0 * dv32 + rr * dv32, cq, Dw, st_[rr]);
        else
            st_[rr][0] = st_[rr][1] = st_[rr][2] = st_[rr][3] = 0.f;
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
            if ((tid & 63) == 0) {
                norm2[0][tid >> 6] = pq;
                norm2[1][tid >> 6] = pk;
            }
        }
        __syncthreads();
        float qmul = scale, kmul = 1.f;
        if (l2norm) {
            // x * (1 / sqrt(sum x^2 + eps)) (recurrent.rs:400-404); the four wavefronts' sums
            // added in a fixed order, so that a call's result does not depend on their timing
            qmul = 1.f / sqrtf(((norm2[0][0] + norm2[0][1]) + (norm2[0][2] + norm2[0][3])) + 1e-6f);
            kmul = 1.f / sqrtf(((norm2[1][0] + norm2[1][1]) + (norm2[1][2] + norm2[1][3])) + 1e-6f);
        }
        const float decay = expf(ld_any(g_dt, g, g_at(a, t, h)));
        const float bt = ld_any(beta_dt, beta, b_at(a, t, h));

        // S <- exp(g) S ; partial S^T k
        float part[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int rr = 0; rr < MAXR; rr++) {
            const int64_t row = r0 + rr;
            const float kr = (ONE || (active && rr < rows_per && row < Dk)) ? ks[row] * kmul : 0.f;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                st_[rr][c] *= decay;
                part[c] += st_[rr][c] * kr;
            }
        }
        if (active)
#pragma unroll
            for (int c = 0; c < 4; c++) red[kg * NQ * 4 + cq + c] = part[c];
        __syncthreads();
        float delta[4];
        const int64_t v_off = v_at(a, t, h) + c0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            float kv = 0.f;
            for (int x = 0; x < NKG; x++) kv += red[x * NQ * 4 + cq + c];
            delta[c] = cq + c < Dw ? (ld<DT>(v, v_off + cq + c) - kv) * bt : 0.f;
        }
        __syncthreads();
        // S <- S + k delta^T ; partial S^T q
#pragma unroll
        for (int c = 0; c < 4; c++) part[c] = 0.f;
#pragma unroll
        for (int rr = 0; rr < MAXR; rr++) {
            const int64_t row = r0 + rr;
            const bool ok = ONE || (active && rr < rows_per && row < Dk);
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
            for (int c = 0; c < 4; c++) red[kg * NQ * 4 + cq + c] = part[c];
        __syncthreads();
        if (kg == 0) {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                float o = 0.f;
                for (int x = 0; x < NKG; x++) o += red[x * NQ * 4 + cq + c];
                if (cq + c < Dw) st<DT>(out, (t * H + h) * Dv + c0 + cq + c, o);
            }
        }
        __syncthreads();
    }

    float *sout = state_out + sh * Dk * Dv + c0;
#pragma unroll
    for (int rr = 0; rr < MAXR; rr++) {
        const int64_t row = r0 + rr;
        if (ONE || (active && rr < rows_per && row < Dk))
            st_cols<VEC>(sout + r0 * dv32 + rr * dv32, cq, Dw, st_[rr]);
    }
}

// ------------------------------------------------------------------------------------------
// The step's backward
// ------------------------------------------------------------------------------------------

// A sum over the 256 threads, the same on every thread, in a fixed order (the four wavefronts'
// sums added in turn). `w4` holds 4 floats of LDS; the call synchronises the workgroup.
__device__ __forceinline__ float block_sum_256(float x, float *w4) {
    x = wave_sum(x);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) w4[threadIdx.x >> 6] = x;
    __syncthreads();
    return (w4[0] + w4[1]) + (w4[2] + w4[3]);
}

// The per-slice partial sums' row: dq_s's Dk, dk's Dk, dg and dbeta, padded to whole 16-byte
// pieces.
__host__ __device__ inline int64_t step_pw(int64_t dk) { return (2 * dk + 2 + 3) & ~(int64_t)3; }

// A sum over the P lanes of a row group (P a power of two dividing 64, the group aligned to P
// lanes), in every lane of the group.
__device__ __forceinline__ float group_sum(float x, int P) {
    for (int o = P >> 1; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
}

// The gradients of the step (the reverse of recurrent.rs:362-396, what the reference's tracked
// step takes from autodiff over the same operations, :89-130). Per token, in reverse, with P the
// state before the token, S' = a P (a = exp g) and S = S' + k delta^T:
//   dS += qs dO^T;  dqs = S dO;  ddelta = dS^T k;  dkv = -beta ddelta;  dv = beta ddelta;
//   dbeta = ddelta . (v - S'^T k);  dk = dS delta + S' dkv;  dS' = dS + k dkv^T;
//   dg = sum(dS' o S');  dP = a dS'.
// One workgroup per (sequence, head, column slice) carries dS for its columns in registers.
// The states before each token past a sequence's first come from a forward sweep that keeps
// them in `states` ([rows, H, Dk, Dv]); the first is state_in. The sums over the columns (dqs,
// dk, dg, dbeta) are per slice, into `part` ([ncs][rows * H][2 Dk + 2]); gdr_step_bwd_finish
// adds the slices and takes them through the scale and the l2 normalisation.
// ONE: one token per sequence (no offsets), Dk = 128 and 64-column slices (16 lanes x 4 columns
// by 16 row groups of 8 rows): every index and bound is then known at compile time.
template <int DT, bool VEC, int MAXR, bool ONE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(ONE ? 3 : 1))) void gdr_step_bwd_kernel(
    GdrArgs a, int64_t rows, int64_t Dk_, int64_t Dv, int ncs, int P_,
    const int32_t *__restrict__ cu, const float *state_in, const float *d_state, float *states,
    const void *d_out, void *dv_out, float *part, float *d_state_in) {
    static_assert(!ONE || (VEC && MAXR == 8), "the one-token form is the 8-row vector one");
    const int64_t Dk = ONE ? 128 : Dk_;
    const int P = ONE ? 16 : P_;
    const int64_t H = a.H;
    const int g_dt = a.g_dt, beta_dt = a.beta_dt, l2norm = a.l2norm;
    const float scale = a.scale;
    const void *q = a.q, *k = a.k, *v = a.v, *g = a.g, *beta = a.beta;
    const int slice = blockIdx.x % ncs;
    const int64_t sh = blockIdx.x / ncs;
    const int64_t s = sh / H, h = sh % H;
    const int64_t Dw = ONE ? 64 : Dv / ncs, c0 = slice * Dw;
    const int tid = threadIdx.x;
    const int NKG = 256 / P;
    const int quad = tid % P, kg = tid / P;
    const int cq = quad * 4;
    const int rows_per = (int)((Dk + NKG - 1) / NKG);
    const int r0 = kg * rows_per;
    const int64_t PW = step_pw(Dk);

    extern __shared__ float sm[];
    float *qsh = sm;           // [Dk] the token's q, f32
    float *ksh = qsh + Dk;     // [Dk] its k
    float *red = ksh + Dk;     // [NKG][4 P] column partial sums
    __shared__ float w4[4];

    const int64_t t0 = !ONE && cu ? cu[s] : s, t1 = !ONE && cu ? cu[s + 1] : s + 1;
    const int64_t DD = Dk * Dv;
    // a row's offset from the slice's first, in 32 bits (Dk x Dv is at most 2^16)
    auto roff = [&](int rr) { return r0 * (int)Dv + rr * (int)Dv; };

    // the token's normalised rows: loads q and k into LDS, returns the multipliers of q (the
    // scale included) and k
    auto load_qk = [&](int64_t t, bool want_q, float &qmul, float &kmul) {
        float pq = 0.f, pk = 0.f;
        const int64_t q_off = q_at(a, t, h), k_off = k_at(a, t, h);
        for (int64_t x = tid; x < Dk; x += 256) {
            const float kv = ld<DT>(k, k_off + x);
            ksh[x] = kv;
            pk += kv * kv;
            if (want_q) {
                const float qv = ld<DT>(q, q_off + x);
                qsh[x] = qv;
                pq += qv * qv;
            }
        }
        qmul = scale, kmul = 1.f;
        if (l2norm) {
            const float sq = block_sum_256(pq, w4);
            const float sk = block_sum_256(pk, w4);
            qmul = scale * (1.f / sqrtf(sq + 1e-6f));
            kmul = 1.f / sqrtf(sk + 1e-6f);
        } else {
            __syncthreads();
        }
    };
    auto row_ok = [&](int rr) { return ONE || (rr < rows_per && r0 + rr < Dk); };
    // the column sums of x[rr][c] * w[row] over the workgroup's rows, for this thread's columns
    auto col_sum = [&](float (*x)[4], const float *w, float wmul, float outv[4]) {
        float p4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int rr = 0; rr < MAXR; rr++) {
            const float wr = row_ok(rr) ? w[r0 + rr] * wmul : 0.f;
#pragma unroll
            for (int c = 0; c < 4; c++) p4[c] += x[rr][c] * wr;
        }
#pragma unroll
        for (int c = 0; c < 4; c++) red[kg * P * 4 + cq + c] = p4[c];
        __syncthreads();
#pragma unroll
        for (int c = 0; c < 4; c++) {
            float acc = 0.f;
            for (int x2 = 0; x2 < NKG; x2++) acc += red[x2 * P * 4 + cq + c];
            outv[c] = acc;
        }
        __syncthreads();
    };

    float racc[MAXR];    // the one-token form: a row group's sums, stored 4 at a time
    float Pst[MAXR][4];  // the state before the token
    float dS[MAXR][4];   // the gradient of the state after it
    const float *sin = state_in + sh * DD + c0;
    auto load_state = [&](const float *base) {
#pragma unroll
        for (int rr = 0; rr < MAXR; rr++) {
            if (row_ok(rr))
                ld_cols<VEC>(base + roff(rr), cq, Dw, Pst[rr]);
            else
                Pst[rr][0] = Pst[rr][1] = Pst[rr][2] = Pst[rr][3] = 0.f;
        }
    };
    load_state(sin);
#pragma unroll
    for (int rr = 0; rr < MAXR; rr++) {
        if (d_state && row_ok(rr))
            ld_cols<VEC>(d_state + sh * DD + c0 + roff(rr), cq, Dw, dS[rr]);
        else
            dS[rr][0] = dS[rr][1] = dS[rr][2] = dS[rr][3] = 0.f;
    }

    // the forward sweep: the state before each token past the first, kept in `states` (each
    // thread reads back only what it wrote)
    for (int64_t t = t0; t + 1 < t1; t++) {
        float qmul, kmul;
        load_qk(t, false, qmul, kmul);
        const float decay = expf(ld_any(g_dt, g, g_at(a, t, h)));
        const float bt = ld_any(beta_dt, beta, b_at(a, t, h));
#pragma unroll
        for (int rr = 0; rr < MAXR; rr++)
#pragma unroll
            for (int c = 0; c < 4; c++) Pst[rr][c] *= decay;
        float kv[4], delta[4];
        col_sum(Pst, ksh, kmul, kv);
        const int64_t v_off = v_at(a, t, h) + c0;
#pragma unroll
        for (int c = 0; c < 4; c++)
            delta[c] = cq + c < Dw ? (ld<DT>(v, v_off + cq + c) - kv[c]) * bt : 0.f;
        float *dst = states + ((t + 1) * H + h) * DD + c0;
#pragma unroll
        for (int rr = 0; rr < MAXR; rr++) {
            if (!row_ok(rr)) continue;
            const float kr = ksh[r0 + rr] * kmul;
#pragma unroll
            for (int c = 0; c < 4; c++) Pst[rr][c] += kr * delta[c];
            st_cols<VEC>(dst + roff(rr), cq, Dw, Pst[rr]);
        }
        __syncthreads();
    }

    // the reverse sweep
    for (int64_t t = t1 - 1; t >= t0; t--) {
        if (t != t1 - 1) load_state(t == t0 ? sin : states + (t * H + h) * DD + c0);
        float qmul, kmul;
        load_qk(t, true, qmul, kmul);
        const float decay = expf(ld_any(g_dt, g, g_at(a, t, h)));
        const float bt = ld_any(beta_dt, beta, b_at(a, t, h));
        // S' = a P
#pragma unroll
        for (int rr = 0; rr < MAXR; rr++)
#pragma unroll
            for (int c = 0; c < 4; c++) Pst[rr][c] *= decay;
        float kv[4], delta[4], vv[4], dO[4];
        col_sum(Pst, ksh, kmul, kv);
        const int64_t v_off = v_at(a, t, h) + c0, o_off = o_at(a, t, h) + c0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const bool cv = ONE || cq + c < Dw;
            vv[c] = cv ? ld<DT>(v, v_off + cq + c) : 0.f;
            delta[c] = (vv[c] - kv[c]) * bt;
            dO[c] = cv && d_out ? ld<DT>(d_out, o_off + cq + c) : 0.f;
        }
        // dS += qs dO^T ; dqs = (S' + k delta^T) dO, over this slice's columns
#pragma unroll
        for (int rr = 0; rr < MAXR; rr++) {
            const bool ok = row_ok(rr);
            const float qr = ok ? qsh[r0 + rr] * qmul : 0.f;
            const float kr = ok ? ksh[r0 + rr] * kmul : 0.f;
            float acc = 0.f;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                dS[rr][c] += qr * dO[c];
                acc += (Pst[rr][c] + kr * delta[c]) * dO[c];
            }
            acc = group_sum(acc, P);
            if (ONE) {
                // the one-token form: a row group's sums in 16-byte stores of 4
                racc[rr] = acc;
                if (rr % 4 == 3 && quad == 0)
                    *(float4 *)(part + ((int64_t)slice * rows * H + t * H + h) * PW + r0 + rr - 3) =
                        make_float4(racc[rr - 3], racc[rr - 2], racc[rr - 1], racc[rr]);
            } else if (ok && quad == 0) {
                part[((int64_t)slice * rows * H + t * H + h) * PW + r0 + rr] = acc;
            }
        }
        // (the one-token form: a row group's 8 sums as two 16-byte stores)

        // ddelta = dS^T k
        float dd[4], dkv[4];
        col_sum(dS, ksh, kmul, dd);
        float db = 0.f;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            dkv[c] = -bt * dd[c];
            if (kg == 0) db += dd[c] * (vv[c] - kv[c]);
        }
        if (kg == 0) {
            const int64_t dv_off = (t * H + h) * Dv + c0;
#pragma unroll
            for (int c = 0; c < 4; c++)
                if (ONE || cq + c < Dw) st<DT>(dv_out, dv_off + cq + c, bt * dd[c]);
        }
        // dk = dS delta + S' dkv ; dS' = dS + k dkv^T ; dg = sum dS' o S' ; dP = a dS'
        float dg = 0.f;
#pragma unroll
        for (int rr = 0; rr < MAXR; rr++) {
            const bool ok = row_ok(rr);
            const float kr = ok ? ksh[r0 + rr] * kmul : 0.f;
            float acc = 0.f;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                acc += dS[rr][c] * delta[c] + Pst[rr][c] * dkv[c];
                const float d1 = dS[rr][c] + kr * dkv[c];
                dg += d1 * Pst[rr][c];
                dS[rr][c] = decay * d1;
            }
            acc = group_sum(acc, P);
            if (ONE) {
                racc[rr] = acc;
                if (rr % 4 == 3 && quad == 0)
                    *(float4 *)(part + ((int64_t)slice * rows * H + t * H + h) * PW + Dk + r0 + rr - 3) =
                        make_float4(racc[rr - 3], racc[rr - 2], racc[rr - 1], racc[rr]);
            } else if (ok && quad == 0) {
                part[((int64_t)slice * rows * H + t * H + h) * PW + Dk + r0 + rr] = acc;
            }
        }

        dg = block_sum_256(dg, w4);
        db = block_sum_256(db, w4);
        if (tid == 0) {
            part[((int64_t)slice * rows * H + t * H + h) * PW + 2 * Dk] = dg;
            part[((int64_t)slice * rows * H + t * H + h) * PW + 2 * Dk + 1] = db;
        }
    }
    if (d_state_in) {
        float *dst = d_state_in + sh * DD + c0;
#pragma unroll
        for (int rr = 0; rr < MAXR; rr++)
            if (row_ok(rr)) st_cols<VEC>(dst + roff(rr), cq, Dw, dS[rr]);
    }
}

// Per (token, head): the slices' partial sums added in order, then dq and dk through the scale
// and the l2 normalisation (d x = (d xn - xn (xn . d xn)) / n, recurrent.rs:400-404), in the
// inputs' dtype; dg and dbeta in theirs.
template <int DT>
__global__ __launch_bounds__(256) void gdr_step_bwd_finish(GdrArgs a, int64_t rows, int ncs,
                                                           const float *part, void *dq, void *dk,
                                                           void *dg, void *dbeta) {
    const int64_t H = a.H, Dk = a.Dk, PW = step_pw(Dk);
    const int64_t th = blockIdx.x, t = th / H, h = th % H;
    const int tid = threadIdx.x;
    __shared__ float w4[4];
    float dqn = 0.f, dkn = 0.f, qv = 0.f, kv = 0.f;
    if (tid < Dk) {
        for (int sl = 0; sl < ncs; sl++) {
            const float *p = part + ((int64_t)sl * rows * H + th) * PW;
            dqn += p[tid];
            dkn += p[Dk + tid];
        }
        dqn *= a.scale;
        qv = ld<DT>(a.q, q_at(a, t, h) + tid);
        kv = ld<DT>(a.k, k_at(a, t, h) + tid);
    }
    if (a.l2norm) {
        const float qi = 1.f / sqrtf(block_sum_256(qv * qv, w4) + 1e-6f);
        const float ki = 1.f / sqrtf(block_sum_256(kv * kv, w4) + 1e-6f);
        const float sq = block_sum_256(qv * qi * dqn, w4);
        const float sk = block_sum_256(kv * ki * dkn, w4);
        dqn = qi * (dqn - qv * qi * sq);
        dkn = ki * (dkn - kv * ki * sk);
    }
    if (tid < Dk) {
        st<DT>(dq, th * Dk + tid, dqn);
        st<DT>(dk, th * Dk + tid, dkn);
    }
    if (tid == 0) {
        float sg = 0.f, sb = 0.f;
        for (int sl = 0; sl < ncs; sl++) {
            const float *p = part + ((int64_t)sl * rows * H + th) * PW;
            sg += p[2 * Dk];
            sb += p[2 * Dk + 1];
        }
        st_any(a.g_dt, dg, th, sg);
        st_any(a.beta_dt, dbeta, th, sb);
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

namespace {

// Columns per workgroup: 64 where Dv allows it (more, shorter workgroups let the state's reads
// and writes of different workgroups overlap).
int step_slices(const dm_gdr_desc *d) {
    return (d->dv >= 128 && d->dv % 64 == 0) ? (int)(d->dv / 64) : 1;
}

int pow2_at_least(int64_t x) {
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}

// The step backward's workspace: the states before each token (only for packed sequences, which
// may hold more than one token), then the per-slice partial sums.
struct StepBwdWs {
    size_t states, part, total;
};
StepBwdWs step_bwd_ws(const dm_gdr_desc *d) {
    auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
    StepBwdWs w;
    const size_t rh = (size_t)d->b * (size_t)d->h;
    w.states = d->cu_seqlens ? up(rh * (size_t)d->dk * (size_t)d->dv * sizeof(float)) : 0;
    w.part = up((size_t)step_slices(d) * rh * (size_t)step_pw(d->dk) * sizeof(float));
    w.total = w.states + w.part;
    return w;
}

}  // namespace

extern "C" int dm_gdr_step(const dm_gdr_desc *d, const void *q, const void *k, const void *v,
                           const void *g, const void *beta, const float *state_in,
                           float *state_out, void *out, void *stream) {
    int rc = check_gdr(d, "gated_delta_step", true);
    if (rc) return rc;
    hipStream_t st = (hipStream_t)stream;
    const int64_t nseq = d->cu_seqlens ? d->nseq : d->b;
    const int ncs = step_slices(d);
    const int64_t blocks = nseq * d->h * ncs;
    if (blocks == 0 || d->dk * d->dv == 0) return DM_OK;
    const int64_t dw = d->dv / ncs;
    const int nq = (int)((dw + 3) / 4);
    const int nkg = 256 / nq;
    const int rows = (int)((d->dk + nkg - 1) / nkg);
    const size_t smem = (size_t)(2 * d->dk + nkg * nq * 4) * sizeof(float);
    // 16-byte state rows: Dv a multiple of 4 and both state pointers aligned
    const bool vec = d->dv % 4 == 0 && aligned_16b(state_in) && aligned_16b(state_out);
    const GdrArgs a = gdr_args(d, q, k, v, g, beta, true);
    // one token per sequence at Dk = 128 in 64-column slices: the compile-time form
    const bool one = !d->cu_seqlens && d->dk == 128 && dw == 64 && rows == 8 && vec;
#define STEP(DT, V, R, O)                                                                    \
    gdr_step_kernel<DT, V, R, O><<<(unsigned)blocks, 256, smem, st>>>(                       \
        a, nseq, d->dk, d->dv, ncs, d->cu_seqlens, state_in, state_out, out)
#define STEP_V(DT, R)                  \
    if (vec) STEP(DT, true, R, false); \
    else STEP(DT, false, R, false);
#define STEP_R(DT)                          \
    if (rows <= 4) { STEP_V(DT, 4) }        \
    else if (one) { STEP(DT, true, 8, true); } \
    else if (rows <= 8) { STEP_V(DT, 8) }   \
    else if (rows <= 16) { STEP_V(DT, 16) } \
    else if (rows <= 32) { STEP_V(DT, 32) } \
    else { STEP_V(DT, 64) }
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
#undef STEP_V
#undef STEP
    probe_add(DM_PROBE_GDR_STEP);
    DM_LAUNCH_CHECK("gated_delta_step: launch");
    return DM_OK;
}

extern "C" size_t dm_gdr_step_bwd_workspace(const dm_gdr_desc *d) {
    if (!d || d->b < 0 || d->h < 0 || d->dk < 0 || d->dv < 0) return 0;
    return step_bwd_ws(d).total;
}

extern "C" int dm_gdr_step_bwd(const dm_gdr_desc *d, const void *q, const void *k,
                               const void *v, const void *g, const void *beta,
                               const float *state_in, const void *d_out, const float *d_state,
                               void *dq, void *dk, void *dv, void *dg, void *dbeta,
                               float *d_state_in, void *workspace, size_t workspace_bytes,
                               void *stream) {
    const char *op = "gated_delta_step_backward";
    int rc = check_gdr(d, op, true);
    if (rc) return rc;
    const StepBwdWs w = step_bwd_ws(d);
    if (workspace_bytes < w.total)
        return refuse(std::string(op) + ": the workspace is smaller than dm_gdr_step_bwd_workspace");
    if (w.total && !workspace) return refuse(std::string(op) + ": null workspace");
    hipStream_t st = (hipStream_t)stream;
    const int64_t nseq = d->cu_seqlens ? d->nseq : d->b;
    const int ncs = step_slices(d);
    const int64_t blocks = nseq * d->h * ncs;
    if (blocks == 0 || d->dk * d->dv == 0) return DM_OK;
    const int64_t dw = d->dv / ncs;
    const int P = pow2_at_least((dw + 3) / 4);  // lanes of a row group, <= 64 for Dv <= 256
    const int nkg = 256 / P;
    const int rows = (int)((d->dk + nkg - 1) / nkg);
    if (rows > 64) return refuse(std::string(op) + ": state shape not implemented");
    const size_t smem = (size_t)(2 * d->dk + nkg * P * 4) * sizeof(float);
    const bool vec = d->dv % 4 == 0 && aligned_16b(state_in) && aligned_16b(d_state) &&
                     aligned_16b(d_state_in) && aligned_16b(workspace);
    float *states = w.states ? (float *)workspace : nullptr;
    float *part = (float *)((char *)workspace + w.states);
    const GdrArgs a = gdr_args(d, q, k, v, g, beta, true);
    const int64_t nrows = d->b;
    // one token per sequence at Dk = 128 in 64-column slices: the compile-time form
    const bool one = !d->cu_seqlens && d->dk == 128 && dw == 64 && P == 16 && rows == 8 && vec;
#define BWD(DT, V, R, O)                                                                     \
    gdr_step_bwd_kernel<DT, V, R, O><<<(unsigned)blocks, 256, smem, st>>>(                   \
        a, nrows, d->dk, d->dv, ncs, P, d->cu_seqlens, state_in, d_state, states, d_out, dv, \
        part, d_state_in)
#define BWD_V(DT, R)                  \
    if (vec) BWD(DT, true, R, false); \
    else BWD(DT, false, R, false);
#define BWD_R(DT)                          \
    if (rows <= 4) { BWD_V(DT, 4) }        \
    else if (one) { BWD(DT, true, 8, true); } \
    else if (rows <= 8) { BWD_V(DT, 8) }   \
    else if (rows <= 16) { BWD_V(DT, 16) } \
    else if (rows <= 32) { BWD_V(DT, 32) } \
    else { BWD_V(DT, 64) }
#define FIN(DT)                                                                                 \
    if (nrows * d->h)                                                                          \
        gdr_step_bwd_finish<DT><<<(unsigned)(nrows * d->h), 256, 0, st>>>(a, nrows, ncs, part, \
                                                                          dq, dk, dg, dbeta);
    {
        KernelTimer timer(DM_KERNEL_GDR_STEP_BWD, st);
        if (d->dtype == DM_F32) {
            BWD_R(DM_F32)
            FIN(DM_F32)
        } else if (d->dtype == DM_BF16) {
            BWD_R(DM_BF16)
            FIN(DM_BF16)
        } else {
            BWD_R(DM_F16)
            FIN(DM_F16)
        }
    }
#undef FIN
#undef BWD_R
#undef BWD_V
#undef BWD
    probe_add(DM_PROBE_GDR_STEP_BWD);
    DM_LAUNCH_CHECK("gated_delta_step_backward: launch");
    return DM_OK;
}
