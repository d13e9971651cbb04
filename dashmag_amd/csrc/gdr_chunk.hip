// The chunked gated delta rule, forward and backward (crates/dash-ops/src/gated_delta/chunk.rs,
// chunk/cube.rs): the plan over packed sequences, and the generic kernel set (any dtype, heads
// up to 256 wide, f32 arithmetic throughout). The MFMA forward for bf16/f16 at Dk = Dv = 128 is
// in gdr_chunk_mfma.hip and is chosen when it takes the call.
//
// Notation per chunk of C = 64 tokens (chunk/reference.rs:11-18), Q already scaled:
//   G = cumsum(g), gamma = exp(G), lam = exp(G_last - G), decay_ij = exp(G_i - G_j) (i >= j)
//   A_ij = beta_i (k_i . k_j) decay_ij (i > j), T = (I + A)^-1
//   W = T (beta gamma K), U = T (beta V), V' = U - W S, O = (gamma Q) S + (Q K^T o decay) V'
//   S_next = exp(G_last) S + (lam K)^T V'.
//
// Launches (forward): plan -> prep (per chunk and head) -> state pass (per sequence and head,
// serial over its chunks) -> output (per chunk and head). Backward: plan -> prep -> state pass
// -> dv_local (per chunk) -> reverse state pass (per sequence) -> gradients (per chunk).
#include <string>

#include "attention_kernels.h"
#include "gdr_common.h"

namespace dm {

// ------------------------------------------------------------------------------------------
// Plan (chunk/cube.rs:80-175): per sequence its first chunk, per chunk its sequence, first
// token and token count. Packed sequences are chunked from their own first token; every chunk
// index up to the host's bound n_max that no sequence uses gets a count of 0.
// ------------------------------------------------------------------------------------------

__global__ __launch_bounds__(1024) void gdr_plan(int64_t nseq, int64_t T, int64_t n_max,
                                                 const int32_t *__restrict__ cu,
                                                 int32_t *__restrict__ seq_chunk0,
                                                 int32_t *__restrict__ chunk_seq,
                                                 int32_t *__restrict__ chunk_tok0,
                                                 int32_t *__restrict__ chunk_len,
                                                 int32_t *__restrict__ seq_order) {
    __shared__ int32_t part[1024];
    const int tid = threadIdx.x;
    const int64_t per = (nseq + 1023) / 1024;
    const int64_t s0 = tid * per, s1 = s0 + per < nseq ? s0 + per : nseq;
    auto span = [&](int64_t s, int64_t *a, int64_t *b) {
        if (cu) {
            *a = cu[s];
            *b = cu[s + 1];
            if (*a < 0) *a = 0;
            if (*b > T) *b = T;  // malformed offsets stay inside the tokens (cube.rs:80-91)
            if (*b < *a) *b = *a;
        } else {
            *a = s * T;
            *b = s * T + T;
        }
    };
    // chunks per thread's sequences, then an inclusive scan over the threads
    int32_t local = 0;
    for (int64_t s = s0; s < s1; s++) {
        int64_t a, b;
        span(s, &a, &b);
        local += (int32_t)((b - a + kChunk - 1) / kChunk);
    }
    part[tid] = local;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {
        const int32_t y = tid >= o ? part[tid - o] : 0;
        __syncthreads();
        part[tid] += y;
        __syncthreads();
    }
    int32_t c = part[tid] - local;
    for (int64_t s = s0; s < s1; s++) {
        int64_t a, b;
        span(s, &a, &b);
        seq_chunk0[s] = c < n_max ? c : (int32_t)n_max;
        c += (int32_t)((b - a + kChunk - 1) / kChunk);
    }
    const int32_t used = part[1023] < n_max ? part[1023] : (int32_t)n_max;
    if (tid == 0) seq_chunk0[nseq] = used;
    __syncthreads();  // (orders the global writes above for the whole workgroup)
    // optionally the sequences by chunk count, the most first (ties by index): the state
    // passes start the longest chains first. Past kOrderMax sequences, the identity.
    if (seq_order) {
        for (int64_t s = tid; s < nseq; s += 1024) {
            if (nseq > kOrderMax) {
                seq_order[s] = (int32_t)s;
                continue;
            }
            const int32_t n = seq_chunk0[s + 1] - seq_chunk0[s];
            int32_t rank = 0;
            for (int64_t u = 0; u < nseq; u++) {
                const int32_t m = seq_chunk0[u + 1] - seq_chunk0[u];
                rank += (m > n) | ((m == n) & (u < s));
            }
            seq_order[rank] = (int32_t)s;
        }
    }
    // every chunk in parallel: its sequence is the last whose first chunk is at or before it
    for (int64_t x = tid; x < n_max; x += 1024) {
        if (x >= used) {
            chunk_seq[x] = 0;
            chunk_tok0[x] = 0;
            chunk_len[x] = 0;
            continue;
        }
        int64_t lo = 0, hi = nseq - 1;  // seq_chunk0[lo] <= x
        while (lo < hi) {
            const int64_t mid = (lo + hi + 1) >> 1;
            if (seq_chunk0[mid] <= x)
                lo = mid;
            else
                hi = mid - 1;
        }
        int64_t a, b;
        span(lo, &a, &b);
        const int64_t t = a + (x - seq_chunk0[lo]) * kChunk;
        chunk_seq[x] = (int32_t)lo;
        chunk_tok0[x] = (int32_t)t;
        chunk_len[x] = (int32_t)(b - t < kChunk ? b - t : kChunk);
    }
}

// ------------------------------------------------------------------------------------------
// Prep (intra, chunk/reference.rs:429-479): per (chunk, head) the normalised and scaled queries
// and keys, G, A, T = (I + A)^-1 by forward substitution, W and U.
// ------------------------------------------------------------------------------------------

template <int DT>
__global__ __launch_bounds__(256) void gdr_prep(GdrArgs a, GdrWs w, int keep_ta) {
    const int64_t ch = blockIdx.x, n = ch / a.H, h = ch % a.H;
    const int len = w.chunk_len[n];
    if (len == 0) return;
    const int64_t tok0 = w.chunk_tok0[n];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t Dk = a.Dk, Dv = a.Dv;
    __shared__ float G[kChunk], gam[kChunk], bet[kChunk];
    __shared__ float Am[kChunk][kChunk + 1], Tm[kChunk][kChunk + 1];
    __shared__ float rowtmp[kChunk];

    float *Qn = w.qn + ch * kChunk * Dk, *Kn = w.kn + ch * kChunk * Dk;
    if (tid < kChunk) {
        const bool ok = tid < len;
        const int64_t t = tok0 + tid;
        G[tid] = ok ? ld_any(a.g_dt, a.g, g_at(a, t, h)) : 0.f;
        bet[tid] = ok ? ld_any(a.beta_dt, a.beta, b_at(a, t, h)) : 0.f;
    }
    // rows: one wavefront per row, lanes along the head
    for (int i = wave; i < kChunk; i += 4) {
        const bool ok = i < len;
        const int64_t qb = q_at(a, tok0 + i, h), kb = k_at(a, tok0 + i, h);
        float sq = 0.f, sk = 0.f;
        for (int64_t x = lane; x < Dk; x += 64) {
            const float qv = ok ? ld<DT>(a.q, qb + x) : 0.f;
            const float kv = ok ? ld<DT>(a.k, kb + x) : 0.f;
            sq += qv * qv;
            sk += kv * kv;
        }
        float qi = 1.f, ki = 1.f;
        if (a.l2norm) {
            qi = 1.f / sqrtf(wave_sum(sq) + 1e-6f);
            ki = 1.f / sqrtf(wave_sum(sk) + 1e-6f);
        }
        for (int64_t x = lane; x < Dk; x += 64) {
            const float qv = ok ? ld<DT>(a.q, qb + x) : 0.f;
            const float kv = ok ? ld<DT>(a.k, kb + x) : 0.f;
            Qn[i * Dk + x] = (a.l2norm ? qv * qi : qv) * a.scale;
            Kn[i * Dk + x] = a.l2norm ? kv * ki : kv;
        }
    }
    __syncthreads();
    if (tid == 0) {
        float acc = 0.f;
        for (int i = 0; i < kChunk; i++) {
            acc += G[i];
            G[i] = acc;
        }
    }
    __syncthreads();
    if (tid < kChunk) {
        gam[tid] = expf(G[tid]);
        w.G[ch * kChunk + tid] = G[tid];
    }
    // A (strictly lower), masked before the exponential
    for (int idx = tid; idx < kChunk * kChunk; idx += 256) {
        const int i = idx / kChunk, j = idx % kChunk;
        float s = 0.f;
        if (i > j) {
            for (int64_t x = 0; x < Dk; x++) s += Kn[i * Dk + x] * Kn[j * Dk + x];
            s = bet[i] * s * expf(G[i] - G[j]);
        }
        Am[i][j] = s;
        Tm[i][j] = -s;
    }
    __syncthreads();
    // forward substitution, one row at a time: row_i += row_i . m[:i, :i]
    for (int i = 1; i < kChunk; i++) {
        if (tid < i) {
            float s = 0.f;
            for (int x = 0; x < i; x++) s += Tm[i][x] * Tm[x][tid];
            rowtmp[tid] = Tm[i][tid] + s;
        }
        __syncthreads();
        if (tid < i) Tm[i][tid] = rowtmp[tid];
        __syncthreads();
    }
    if (tid < kChunk) Tm[tid][tid] += 1.f;
    __syncthreads();
    if (keep_ta) {
        for (int idx = tid; idx < kChunk * kChunk; idx += 256) {
            w.Tm[ch * kChunk * kChunk + idx] = Tm[idx / kChunk][idx % kChunk];
            w.Am[ch * kChunk * kChunk + idx] = Am[idx / kChunk][idx % kChunk];
        }
    }
    // W = T (beta gamma K), U = T (beta V)
    float *W = w.W + ch * kChunk * Dk, *U = w.U + ch * kChunk * Dv;
    for (int64_t idx = tid; idx < kChunk * Dk; idx += 256) {
        const int i = (int)(idx / Dk);
        const int64_t x = idx % Dk;
        float s = 0.f;
        for (int j = 0; j <= i; j++) s += Tm[i][j] * (Kn[j * Dk + x] * bet[j] * gam[j]);
        W[idx] = s;
    }
    for (int64_t idx = tid; idx < kChunk * Dv; idx += 256) {
        const int i = (int)(idx / Dv);
        const int64_t y = idx % Dv;
        float s = 0.f;
        for (int j = 0; j <= i && j < len; j++)
            s += Tm[i][j] * (ld<DT>(a.v, v_at(a, tok0 + j, h) + y) * bet[j]);
        U[idx] = s;
    }
}

// ------------------------------------------------------------------------------------------
// State pass (state_forward, chunk/reference.rs:348-372): per (sequence, head), serial over its
// chunks; stores each chunk's entering state and V'.
// ------------------------------------------------------------------------------------------

__global__ __launch_bounds__(256) void gdr_state_fwd(GdrArgs a, GdrWs w, const float *h0,
                                                     float *final_state) {
    const int64_t sh = blockIdx.x, s = sh / a.H, h = sh % a.H;
    const int tid = threadIdx.x;
    const int64_t Dk = a.Dk, Dv = a.Dv, SS = Dk * Dv;
    const int c0 = w.seq_chunk0[s], c1 = w.seq_chunk0[s + 1];
    const float *init = h0 ? h0 + sh * SS : nullptr;
    if (c0 == c1) {
        if (final_state)
            for (int64_t x = tid; x < SS; x += 256) final_state[sh * SS + x] = init ? init[x] : 0.f;
        return;
    }
    float *S0 = w.Sc + ((int64_t)c0 * a.H + h) * SS;
    for (int64_t x = tid; x < SS; x += 256) S0[x] = init ? init[x] : 0.f;
    __syncthreads();
    for (int c = c0; c < c1; c++) {
        const int64_t ch = (int64_t)c * a.H + h;
        const float *S = w.Sc + ch * SS, *W = w.W + ch * kChunk * Dk, *U = w.U + ch * kChunk * Dv;
        const float *Kn = w.kn + ch * kChunk * Dk, *G = w.G + ch * kChunk;
        float *Vn = w.Vn + ch * kChunk * Dv;
        for (int64_t idx = tid; idx < kChunk * Dv; idx += 256) {
            const int i = (int)(idx / Dv);
            const int64_t y = idx % Dv;
            float acc = 0.f;
            for (int64_t x = 0; x < Dk; x++) acc += W[i * Dk + x] * S[x * Dv + y];
            Vn[idx] = U[idx] - acc;
        }
        __syncthreads();
        float *Sn = c + 1 < c1 ? w.Sc + (ch + a.H) * SS : (final_state ? final_state + sh * SS : nullptr);
        if (Sn) {
            const float gl = expf(G[kChunk - 1]);
            for (int64_t idx = tid; idx < SS; idx += 256) {
                const int64_t x = idx / Dv, y = idx % Dv;
                float acc = 0.f;
                for (int i = 0; i < kChunk; i++)
                    acc += Kn[i * Dk + x] * expf(G[kChunk - 1] - G[i]) * Vn[i * Dv + y];
                Sn[idx] = S[idx] * gl + acc;
            }
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------------------------------
// Output (forward, chunk/reference.rs:502-508): O = (gamma Q) S + (Q K^T o decay) V'.
// ------------------------------------------------------------------------------------------

template <int DT>
__global__ __launch_bounds__(256) void gdr_output(GdrArgs a, GdrWs w, void *out) {
    const int64_t ch = blockIdx.x, n = ch / a.H, h = ch % a.H;
    const int len = w.chunk_len[n];
    if (len == 0) return;
    const int64_t tok0 = w.chunk_tok0[n];
    const int tid = threadIdx.x;
    const int64_t Dk = a.Dk, Dv = a.Dv;
    __shared__ float P[kChunk][kChunk + 1];
    __shared__ float G[kChunk];
    const float *Qn = w.qn + ch * kChunk * Dk, *Kn = w.kn + ch * kChunk * Dk;
    const float *S = w.Sc + ch * Dk * Dv, *Vn = w.Vn + ch * kChunk * Dv;
    if (tid < kChunk) G[tid] = w.G[ch * kChunk + tid];
    __syncthreads();
    for (int idx = tid; idx < kChunk * kChunk; idx += 256) {
        const int i = idx / kChunk, j = idx % kChunk;
        float s = 0.f;
        if (i >= j) {
            for (int64_t x = 0; x < Dk; x++) s += Qn[i * Dk + x] * Kn[j * Dk + x];
            s *= expf(G[i] - G[j]);
        }
        P[i][j] = s;
    }
    __syncthreads();
    for (int64_t idx = tid; idx < (int64_t)len * Dv; idx += 256) {
        const int i = (int)(idx / Dv);
        const int64_t y = idx % Dv;
        float inter = 0.f, intra = 0.f;
        for (int64_t x = 0; x < Dk; x++) inter += Qn[i * Dk + x] * S[x * Dv + y];
        for (int j = 0; j <= i; j++) intra += P[i][j] * Vn[j * Dv + y];
        st<DT>(out, ((tok0 + i) * a.H + h) * Dv + y, inter * expf(G[i]) + intra);
    }
}

// ------------------------------------------------------------------------------------------
// Backward (chunk/reference.rs:519-695)
// ------------------------------------------------------------------------------------------

// dv_local = (Q K^T o decay)^T dO, per chunk.
template <int DT>
__global__ __launch_bounds__(256) void gdr_dvlocal(GdrArgs a, GdrWs w, const void *d_out) {
    const int64_t ch = blockIdx.x, n = ch / a.H, h = ch % a.H;
    const int len = w.chunk_len[n];
    if (len == 0) return;
    const int64_t tok0 = w.chunk_tok0[n];
    const int tid = threadIdx.x;
    const int64_t Dk = a.Dk, Dv = a.Dv;
    __shared__ float P[kChunk][kChunk + 1];
    __shared__ float G[kChunk];
    const float *Qn = w.qn + ch * kChunk * Dk, *Kn = w.kn + ch * kChunk * Dk;
    if (tid < kChunk) G[tid] = w.G[ch * kChunk + tid];
    __syncthreads();
    for (int idx = tid; idx < kChunk * kChunk; idx += 256) {
        const int i = idx / kChunk, j = idx % kChunk;
        float s = 0.f;
        if (i >= j) {
            for (int64_t x = 0; x < Dk; x++) s += Qn[i * Dk + x] * Kn[j * Dk + x];
            s *= expf(G[i] - G[j]);
        }
        P[i][j] = s;
    }
    __syncthreads();
    float *dvl = w.dvl + ch * kChunk * Dv;
    for (int64_t idx = tid; idx < kChunk * Dv; idx += 256) {
        const int j = (int)(idx / Dv);
        const int64_t y = idx % Dv;
        float s = 0.f;
        for (int i = j; i < len; i++) s += P[i][j] * ld<DT>(d_out, o_at(a, tok0 + i, h) + y);
        dvl[idx] = s;
    }
}

// state_backward (chunk/reference.rs:382-427), per (sequence, head), reverse over its chunks:
//   dV'_c = (lam K)_c dS_{c+1} + dv_local_c ; dS_c = exp(G_last) dS_{c+1} + (gamma Q)^T dO - W^T dV'.
template <int DT>
__global__ __launch_bounds__(256) void gdr_state_bwd(GdrArgs a, GdrWs w, const void *d_out,
                                                     const float *d_final, float *dh0) {
    const int64_t sh = blockIdx.x, s = sh / a.H, h = sh % a.H;
    const int tid = threadIdx.x;
    const int64_t Dk = a.Dk, Dv = a.Dv, SS = Dk * Dv;
    const int c0 = w.seq_chunk0[s], c1 = w.seq_chunk0[s + 1];
    float *ds = w.ds + sh * SS;
    for (int64_t x = tid; x < SS; x += 256) ds[x] = d_final ? d_final[sh * SS + x] : 0.f;
    __syncthreads();
    for (int c = c1 - 1; c >= c0; c--) {
        const int64_t ch = (int64_t)c * a.H + h;
        const int len = w.chunk_len[c];
        const int64_t tok0 = w.chunk_tok0[c];
        const float *Kn = w.kn + ch * kChunk * Dk, *Qn = w.qn + ch * kChunk * Dk;
        const float *W = w.W + ch * kChunk * Dk, *G = w.G + ch * kChunk;
        const float *dvl = w.dvl + ch * kChunk * Dv;
        float *dSn = w.dSn + ch * SS, *dVn = w.dVn + ch * kChunk * Dv;
        for (int64_t x = tid; x < SS; x += 256) dSn[x] = ds[x];
        const float gl = expf(G[kChunk - 1]);
        for (int64_t idx = tid; idx < kChunk * Dv; idx += 256) {
            const int i = (int)(idx / Dv);
            const int64_t y = idx % Dv;
            const float lam = expf(G[kChunk - 1] - G[i]);
            float acc = 0.f;
            for (int64_t x = 0; x < Dk; x++) acc += Kn[i * Dk + x] * lam * ds[x * Dv + y];
            dVn[idx] = acc + dvl[idx];
        }
        __syncthreads();
        for (int64_t idx = tid; idx < SS; idx += 256) {
            const int64_t x = idx / Dv, y = idx % Dv;
            float qdo = 0.f, wdv = 0.f;
            for (int i = 0; i < kChunk; i++) {
                const float d_o = i < len ? ld<DT>(d_out, o_at(a, tok0 + i, h) + y) : 0.f;
                qdo += Qn[i * Dk + x] * expf(G[i]) * d_o;
                wdv += W[i * Dk + x] * dVn[i * Dv + y];
            }
            ds[idx] = ds[idx] * gl + qdo - wdv;
        }
        __syncthreads();
    }
    if (dh0)
        for (int64_t x = tid; x < SS; x += 256) dh0[sh * SS + x] = ds[x];
}

// Every input's gradient within one chunk (chunk/reference.rs:568-695).
template <int DT>
__global__ __launch_bounds__(256) void gdr_grads(GdrArgs a, GdrWs w, const void *d_out,
                                                 void *dq, void *dk, void *dv, void *dg,
                                                 void *dbeta) {
    const int64_t ch = blockIdx.x, n = ch / a.H, h = ch % a.H;
    const int len = w.chunk_len[n];
    if (len == 0) return;
    const int64_t tok0 = w.chunk_tok0[n];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t Dk = a.Dk, Dv = a.Dv, SS = Dk * Dv;
    constexpr int C = kChunk;
    extern __shared__ float smem[];
    float(*P)[C + 1] = (float(*)[C + 1])smem;              // attn, later m
    float(*DP)[C + 1] = (float(*)[C + 1])(smem + 1 * C * (C + 1));  // d_attn
    float(*DT_)[C + 1] = (float(*)[C + 1])(smem + 2 * C * (C + 1));  // dT
    float(*M1)[C + 1] = (float(*)[C + 1])(smem + 3 * C * (C + 1));   // T^T dT
    float(*DA)[C + 1] = (float(*)[C + 1])(smem + 4 * C * (C + 1));   // dA
    float *G = smem + 5 * C * (C + 1);
    float *gam = G + C, *lam = gam + C, *bet = lam + C, *dgam = bet + C, *dgv = dgam + C,
          *dbv = dgv + C, *red = dbv + C;

    const float *Qn = w.qn + ch * C * Dk, *Kn = w.kn + ch * C * Dk;
    const float *S = w.Sc + ch * SS, *dSn = w.dSn + ch * SS;
    const float *Vn = w.Vn + ch * C * Dv, *dVn = w.dVn + ch * C * Dv;
    const float *Tm = w.Tm + ch * C * C, *Am = w.Am + ch * C * C;
    float *DQ = w.gq + ch * C * Dk, *DK = w.gk + ch * C * Dk, *X = w.gx + ch * C * (Dk > Dv ? Dk : Dv);
    auto dO = [&](int i, int64_t y) -> float {
        return i < len ? ld<DT>(d_out, o_at(a, tok0 + i, h) + y) : 0.f;
    };
    auto Vin = [&](int i, int64_t y) -> float {
        return i < len ? ld<DT>(a.v, v_at(a, tok0 + i, h) + y) : 0.f;
    };
    if (tid < C) {
        G[tid] = w.G[ch * C + tid];
        bet[tid] = tid < len ? ld_any(a.beta_dt, a.beta, b_at(a, tok0 + tid, h)) : 0.f;
    }
    __syncthreads();
    if (tid < C) {
        gam[tid] = expf(G[tid]);
        lam[tid] = expf(G[C - 1] - G[tid]);
    }
    const float gl = expf(G[C - 1]);
    // attn = (Q K^T) o decay ; d_attn = (dO V'^T) o incl
    for (int idx = tid; idx < C * C; idx += 256) {
        const int i = idx / C, j = idx % C;
        float s = 0.f, d = 0.f;
        if (i >= j) {
            for (int64_t x = 0; x < Dk; x++) s += Qn[i * Dk + x] * Kn[j * Dk + x];
            s *= expf(G[i] - G[j]);
            for (int64_t y = 0; y < Dv; y++) d += dO(i, y) * Vn[j * Dv + y];
        }
        P[i][j] = s;
        DP[i][j] = d;
    }
    __syncthreads();
    // d_qg = dO S^T: dq = d_qg gamma; d_gamma = rowsum(d_qg Q)
    for (int64_t idx = tid; idx < C * Dk; idx += 256) {
        const int i = (int)(idx / Dk);
        const int64_t x = idx % Dk;
        float s = 0.f;
        for (int64_t y = 0; y < Dv; y++) s += dO(i, y) * S[x * Dv + y];
        X[idx] = s;
        DQ[idx] = s * gam[i];
    }
    __syncthreads();
    for (int i = wave; i < C; i += 4) {
        float s = 0.f;
        for (int64_t x = lane; x < Dk; x += 64) s += X[i * Dk + x] * Qn[i * Dk + x];
        s = wave_sum(s);
        if (lane == 0) dgam[i] = s;
    }
    // dq += (d_attn o decay) K ; dk = (d_attn o decay)^T Q
    for (int64_t idx = tid; idx < C * Dk; idx += 256) {
        const int i = (int)(idx / Dk);
        const int64_t x = idx % Dk;
        float sq = 0.f, sk = 0.f;
        for (int j = 0; j <= i; j++) sq += DP[i][j] * expf(G[i] - G[j]) * Kn[j * Dk + x];
        for (int j = i; j < C; j++) sk += DP[j][i] * expf(G[j] - G[i]) * Qn[j * Dk + x];
        DQ[idx] += sq;
        DK[idx] = sk;
    }
    __syncthreads();
    // m = d_attn o attn: d_g = rowsum(m) - colsum(m)
    if (tid < C) {
        float rs = 0.f, cs = 0.f;
        for (int j = 0; j < C; j++) {
            rs += DP[tid][j] * P[tid][j];
            cs += DP[j][tid] * P[j][tid];
        }
        dgv[tid] = rs - cs;
    }
    __syncthreads();
    // d_kt = V' dS_next^T: dk += d_kt lam; lam_dlam = lam rowsum(d_kt K); d_g -= lam_dlam
    for (int64_t idx = tid; idx < C * Dk; idx += 256) {
        const int i = (int)(idx / Dk);
        const int64_t x = idx % Dk;
        float s = 0.f;
        for (int64_t y = 0; y < Dv; y++) s += Vn[i * Dv + y] * dSn[x * Dv + y];
        X[idx] = s;
        DK[idx] += s * lam[i];
    }
    __syncthreads();
    for (int i = wave; i < C; i += 4) {
        float s = 0.f;
        for (int64_t x = lane; x < Dk; x += 64) s += X[i * Dk + x] * Kn[i * Dk + x];
        s = wave_sum(s);
        if (lane == 0) {
            const float ld_ = s * lam[i];
            dgv[i] -= ld_;
            red[i] = ld_;
        }
    }
    // s_ds = sum(S o dS_next)
    float part = 0.f;
    for (int64_t x = tid; x < SS; x += 256) part += S[x] * dSn[x];
    part = wave_sum(part);
    __syncthreads();
    if (lane == 0) red[C + wave] = part;
    __syncthreads();
    if (tid == 0) {
        float lsum = 0.f;
        for (int i = 0; i < C; i++) lsum += red[i];
        const float s_ds = red[C] + red[C + 1] + red[C + 2] + red[C + 3];
        dgv[C - 1] += lsum + s_ds * gl;
    }
    __syncthreads();
    // dw = -(dV' S^T) into X ; dT = dV' (beta V)^T + dw (beta gamma K)^T
    for (int64_t idx = tid; idx < C * Dk; idx += 256) {
        const int i = (int)(idx / Dk);
        const int64_t x = idx % Dk;
        float s = 0.f;
        for (int64_t y = 0; y < Dv; y++) s += dVn[i * Dv + y] * S[x * Dv + y];
        X[idx] = -s;
    }
    __syncthreads();
    for (int idx = tid; idx < C * C; idx += 256) {
        const int i = idx / C, j = idx % C;
        float s = 0.f;
        for (int64_t y = 0; y < Dv; y++) s += dVn[i * Dv + y] * Vin(j, y);
        s *= bet[j];
        float s2 = 0.f;
        for (int64_t x = 0; x < Dk; x++) s2 += X[i * Dk + x] * Kn[j * Dk + x];
        DT_[i][j] = s + s2 * bet[j] * gam[j];
    }
    __syncthreads();
    // d_vb = T^T dV': dv = d_vb beta ; d_beta = rowsum(d_vb V)
    if (tid < C) dbv[tid] = 0.f;
    __syncthreads();
    for (int64_t idx = tid; idx < (int64_t)len * Dv; idx += 256) {
        const int i = (int)(idx / Dv);
        const int64_t y = idx % Dv;
        float s = 0.f;
        for (int j = i; j < C; j++) s += Tm[j * C + i] * dVn[j * Dv + y];
        st<DT>(dv, ((tok0 + i) * a.H + h) * Dv + y, s * bet[i]);
    }
    for (int i = wave; i < C; i += 4) {
        float acc = 0.f;
        for (int64_t y = lane; y < Dv; y += 64) {
            float s = 0.f;
            for (int j = i; j < C; j++) s += Tm[j * C + i] * dVn[j * Dv + y];
            acc += s * Vin(i, y);
        }
        acc = wave_sum(acc);
        if (lane == 0) dbv[i] = acc;
    }
    __syncthreads();
    // d_kbg = T^T dw: d_beta += rowsum(d_kbg K gamma); dk += d_kbg beta gamma;
    // d_gamma += rowsum(d_kbg K beta)
    for (int i = wave; i < C; i += 4) {
        float s2 = 0.f;
        for (int64_t x = lane; x < Dk; x += 64) {
            float s = 0.f;
            for (int j = i; j < C; j++) s += Tm[j * C + i] * X[j * Dk + x];
            s2 += s * Kn[i * Dk + x];
            DK[i * Dk + x] += s * bet[i] * gam[i];
        }
        s2 = wave_sum(s2);
        if (lane == 0) {
            dbv[i] += s2 * gam[i];
            dgam[i] += s2 * bet[i];
        }
    }
    __syncthreads();
    if (tid < C) dgv[tid] += dgam[tid] * gam[tid];
    // dA = -(T^T dT T^T), strictly lower
    for (int idx = tid; idx < C * C; idx += 256) {
        const int i = idx / C, j = idx % C;
        float s = 0.f;
        for (int x = 0; x < C; x++) s += Tm[x * C + i] * DT_[x][j];
        M1[i][j] = s;
    }
    __syncthreads();
    for (int idx = tid; idx < C * C; idx += 256) {
        const int i = idx / C, j = idx % C;
        float s = 0.f;
        if (i > j)
            for (int x = 0; x < C; x++) s += M1[i][x] * Tm[j * C + x];
        DA[i][j] = -s;
    }
    __syncthreads();
    // A = (beta K K^T) o decay, strictly lower: dae = dA o decay
    for (int idx = tid; idx < C * C; idx += 256) {
        const int i = idx / C, j = idx % C;
        P[i][j] = i > j ? DA[i][j] * expf(G[i] - G[j]) : 0.f;
    }
    __syncthreads();
    // d_kbeta = dae K: dk += d_kbeta beta ; d_beta += rowsum(d_kbeta K) ; dk += dae^T (K beta)
    for (int i = wave; i < C; i += 4) {
        float s2 = 0.f;
        for (int64_t x = lane; x < Dk; x += 64) {
            float s = 0.f, t = 0.f;
            for (int j = 0; j < i; j++) s += P[i][j] * Kn[j * Dk + x];
            for (int j = i + 1; j < C; j++) t += P[j][i] * Kn[j * Dk + x] * bet[j];
            s2 += s * Kn[i * Dk + x];
            DK[i * Dk + x] += s * bet[i] + t;
        }
        s2 = wave_sum(s2);
        if (lane == 0) dbv[i] += s2;
    }
    __syncthreads();
    // m = dA o A: d_g += rowsum - colsum ; then the reverse cumulative sum
    if (tid < C) {
        float rs = 0.f, cs = 0.f;
        for (int j = 0; j < C; j++) {
            rs += DA[tid][j] * Am[tid * C + j];
            cs += DA[j][tid] * Am[j * C + tid];
        }
        dgv[tid] += rs - cs;
    }
    __syncthreads();
    if (tid == 0) {
        float tail = 0.f;
        for (int i = C - 1; i >= 0; i--) {
            tail += dgv[i];
            red[i] = tail;
        }
    }
    __syncthreads();
    if (tid < len) {
        st_any(a.g_dt, dg, (tok0 + tid) * a.H + h, red[tid]);
        st_any(a.beta_dt, dbeta, (tok0 + tid) * a.H + h, dbv[tid]);
    }
    // dq (scaled), dk, through the l2 normalisation (l2norm_backward :246-252)
    for (int i = wave; i < len; i += 4) {
        const int64_t base = ((tok0 + i) * a.H + h) * Dk;  // the gradients' (contiguous)
        const int64_t qb = q_at(a, tok0 + i, h), kb = k_at(a, tok0 + i, h);
        float qi = 1.f, ki = 1.f, sq = 0.f, sk = 0.f;
        if (a.l2norm) {
            float nq = 0.f, nk = 0.f;
            for (int64_t x = lane; x < Dk; x += 64) {
                const float qv = ld<DT>(a.q, qb + x), kv = ld<DT>(a.k, kb + x);
                nq += qv * qv;
                nk += kv * kv;
            }
            qi = 1.f / sqrtf(wave_sum(nq) + 1e-6f);
            ki = 1.f / sqrtf(wave_sum(nk) + 1e-6f);
            for (int64_t x = lane; x < Dk; x += 64) {
                sq += ld<DT>(a.q, qb + x) * qi * DQ[i * Dk + x] * a.scale;
                sk += ld<DT>(a.k, kb + x) * ki * DK[i * Dk + x];
            }
            sq = wave_sum(sq);
            sk = wave_sum(sk);
        }
        for (int64_t x = lane; x < Dk; x += 64) {
            const float gq = DQ[i * Dk + x] * a.scale, gk = DK[i * Dk + x];
            if (a.l2norm) {
                st<DT>(dq, base + x, qi * (gq - ld<DT>(a.q, qb + x) * qi * sq));
                st<DT>(dk, base + x, ki * (gk - ld<DT>(a.k, kb + x) * ki * sk));
            } else {
                st<DT>(dq, base + x, gq);
                st<DT>(dk, base + x, gk);
            }
        }
    }
}

static size_t grads_smem() { return (5 * kChunk * (kChunk + 1) + 8 * kChunk + 8) * sizeof(float); }

// ------------------------------------------------------------------------------------------
// Host side
// ------------------------------------------------------------------------------------------

int64_t gdr_nseq(const dm_gdr_desc *d) { return d->cu_seqlens ? d->nseq : d->b; }

int64_t gdr_chunk_bound(const dm_gdr_desc *d) {
    if (d->cu_seqlens) return (d->t + (kChunk - 1) * d->nseq) / kChunk;
    return d->b * ((d->t + kChunk - 1) / kChunk);
}

// Carves the workspace; returns the bytes needed (layout identical when `base` is null).
size_t gdr_ws_layout(const dm_gdr_desc *d, bool backward, char *base, GdrWs *w) {
    const int64_t nc = gdr_chunk_bound(d), S = gdr_nseq(d), H = d->h;
    const int64_t Dk = d->dk, Dv = d->dv, C = kChunk, ch = nc * H;
    size_t off = 0;
    auto take = [&](size_t bytes) -> char * {
        char *p = base ? base + off : nullptr;
        off += align_up(bytes);
        return p;
    };
    GdrWs x{};
    x.seq_chunk0 = (int32_t *)take((S + 1) * 4);
    x.chunk_seq = (int32_t *)take(nc * 4);
    x.chunk_tok0 = (int32_t *)take(nc * 4);
    x.chunk_len = (int32_t *)take(nc * 4);
    x.G = (float *)take(ch * C * 4);
    x.qn = (float *)take(ch * C * Dk * 4);
    x.kn = (float *)take(ch * C * Dk * 4);
    x.W = (float *)take(ch * C * Dk * 4);
    x.U = (float *)take(ch * C * Dv * 4);
    x.Sc = (float *)take(ch * Dk * Dv * 4);
    x.Vn = (float *)take(ch * C * Dv * 4);
    if (backward) {
        x.Tm = (float *)take(ch * C * C * 4);
        x.Am = (float *)take(ch * C * C * 4);
        x.dvl = (float *)take(ch * C * Dv * 4);
        x.dSn = (float *)take(ch * Dk * Dv * 4);
        x.dVn = (float *)take(ch * C * Dv * 4);
        x.ds = (float *)take(S * H * Dk * Dv * 4);
        x.gq = (float *)take(ch * C * Dk * 4);
        x.gk = (float *)take(ch * C * Dk * 4);
        x.gx = (float *)take(ch * C * (Dk > Dv ? Dk : Dv) * 4);
    }
    if (w) *w = x;
    return off;
}

bool gdr_strides_ok(const dm_gdr_desc *d, bool step) {
    if (!d->strided) return true;
    const int64_t T = step ? 1 : d->t;
    for (const dm_strides *x : {&d->sq, &d->sk, &d->sv, &d->sg, &d->sbeta, &d->sdo}) {
        if (x->b < 0 || x->t < 0 || x->h < 0) return false;
        if (!step && d->b > 1 && x->b != T * x->t) return false;
    }
    return true;
}

bool gdr_strides_16b(const dm_gdr_desc *d) {
    if (!d->strided) return true;
    for (const dm_strides *x : {&d->sq, &d->sk, &d->sv, &d->sdo})
        if (x->b % 8 || x->t % 8 || x->h % 8) return false;
    return true;
}

GdrArgs gdr_args(const dm_gdr_desc *d, const void *q, const void *k, const void *v,
                 const void *g, const void *beta, bool step) {
    GdrArgs a;
    // contiguous rows unless given: [rows, H, D] and [rows, H]; the step's rows are its batch
    // (t stride = b stride)
    const int64_t H = d->h;
    a.q_t = a.k_t = H * d->dk, a.q_h = a.k_h = d->dk;
    a.v_t = a.o_t = H * d->dv, a.v_h = a.o_h = d->dv;
    a.g_t = a.b_t = H, a.g_h = a.b_h = 1;
    if (d->strided) {
        auto rowst = [&](const dm_strides &x) { return step ? x.b : x.t; };
        a.q_t = rowst(d->sq), a.q_h = d->sq.h;
        a.k_t = rowst(d->sk), a.k_h = d->sk.h;
        a.v_t = rowst(d->sv), a.v_h = d->sv.h;
        a.g_t = rowst(d->sg), a.g_h = d->sg.h;
        a.b_t = rowst(d->sbeta), a.b_h = d->sbeta.h;
        a.o_t = rowst(d->sdo), a.o_h = d->sdo.h;
    }
    a.H = d->h;
    a.rows = d->b * d->t;
    a.Dk = d->dk;
    a.Dv = d->dv;
    a.g_dt = d->g_dtype;
    a.beta_dt = d->beta_dtype;
    a.l2norm = d->qk_l2norm;
    a.scale = d->has_scale ? d->scale : (float)(1.0 / std::sqrt((double)d->dk));
    a.q = q;
    a.k = k;
    a.v = v;
    a.g = g;
    a.beta = beta;
    return a;
}

int launch_plan(const dm_gdr_desc *d, int32_t *seq_chunk0, int32_t *chunk_seq,
                int32_t *chunk_tok0, int32_t *chunk_len, hipStream_t st, int32_t *seq_order) {
    const int64_t nc = gdr_chunk_bound(d), S = gdr_nseq(d);
    gdr_plan<<<1, 1024, 0, st>>>(S, d->t, nc, d->cu_seqlens, seq_chunk0, chunk_seq, chunk_tok0,
                                chunk_len, seq_order);
    DM_LAUNCH_CHECK("chunk_gated_delta_rule: plan");
    return DM_OK;
}

int launch_gdr_plan(const dm_gdr_desc *d, GdrWs &w, hipStream_t st) {
    return launch_plan(d, w.seq_chunk0, w.chunk_seq, w.chunk_tok0, w.chunk_len, st);
}

}  // namespace dm

using namespace dm;

extern "C" {

size_t dm_gdr_chunk_fwd_workspace(const dm_gdr_desc *d) {
    if (!d) return 0;
    if (gdr_mfma_takes(d)) return gdr_mfma_fwd_workspace(d);
    return gdr_ws_layout(d, false, nullptr, nullptr);
}

int dm_gdr_chunk_fwd(const dm_gdr_desc *d, const void *q, const void *k, const void *v,
                     const void *g, const void *beta, const float *h0, void *out,
                     float *final_state, void *workspace, size_t workspace_bytes, void *stream) {
    int rc = check_gdr(d, "chunk_gated_delta_rule", false);
    if (rc) return rc;
    if (workspace_bytes < dm_gdr_chunk_fwd_workspace(d))
        return refuse("chunk_gated_delta_rule: the workspace is smaller than "
                      "dm_gdr_chunk_fwd_workspace");
    hipStream_t st = (hipStream_t)stream;
    const int64_t S = gdr_nseq(d), nc = gdr_chunk_bound(d);
    if (S * d->h == 0) return DM_OK;
    if (gdr_mfma_takes(d)) {
        for (const void *p : {q, k, v, (const void *)out})
            if (!aligned_16b(p))
                return refuse("chunk_gated_delta_rule: q, k, v and out must be 16-byte aligned "
                              "(16-bit heads that are multiples of 8 wide read and write whole "
                              "rows; the host copies other views)");
        return launch_gdr_mfma_fwd(d, q, k, v, g, beta, h0, out, final_state, workspace, st);
    }
    GdrWs w;
    gdr_ws_layout(d, false, (char *)workspace, &w);
    GdrArgs a = gdr_args(d, q, k, v, g, beta);
    if ((rc = launch_gdr_plan(d, w, st))) return rc;
    const unsigned chunks = (unsigned)(nc * d->h);
#define FWD(DT)                                                                 \
    if (chunks) gdr_prep<DT><<<chunks, 256, 0, st>>>(a, w, 0);                  \
    gdr_state_fwd<<<(unsigned)(S * d->h), 256, 0, st>>>(a, w, h0, final_state); \
    if (chunks) gdr_output<DT><<<chunks, 256, 0, st>>>(a, w, out);
    if (d->dtype == DM_F32) {
        FWD(DM_F32)
    } else if (d->dtype == DM_BF16) {
        FWD(DM_BF16)
    } else {
        FWD(DM_F16)
    }
#undef FWD
    probe_add(DM_PROBE_GDR_CHUNK_FWD, 4);
    DM_LAUNCH_CHECK("chunk_gated_delta_rule: launch");
    return DM_OK;
}

size_t dm_gdr_chunk_bwd_workspace(const dm_gdr_desc *d) {
    if (!d) return 0;
    if (gdr_mfma_takes(d)) return gdr_mfma_bwd_workspace(d);
    return gdr_ws_layout(d, true, nullptr, nullptr);
}

int dm_gdr_chunk_bwd(const dm_gdr_desc *d, const void *q, const void *k, const void *v,
                     const void *g, const void *beta, const float *h0, const void *d_out,
                     const float *d_final, void *dq, void *dk, void *dv, void *dg, void *dbeta,
                     float *dh0, void *workspace, size_t workspace_bytes, void *stream) {
    int rc = check_gdr(d, "chunk_gated_delta_rule_backward", false);
    if (rc) return rc;
    if (workspace_bytes < dm_gdr_chunk_bwd_workspace(d))
        return refuse("chunk_gated_delta_rule_backward: the workspace is smaller than "
                      "dm_gdr_chunk_bwd_workspace");
    hipStream_t st = (hipStream_t)stream;
    const int64_t S = gdr_nseq(d), nc = gdr_chunk_bound(d);
    if (S * d->h == 0) return DM_OK;
    if (gdr_mfma_takes(d)) {
        for (const void *p : {q, k, v, d_out, (const void *)dq, (const void *)dk, (const void *)dv})
            if (!aligned_16b(p))
                return refuse("chunk_gated_delta_rule_backward: q, k, v, d_out, dq, dk and dv "
                              "must be 16-byte aligned (16-bit heads that are multiples of 8 "
                              "wide read and write whole rows; the host copies other views)");
        return launch_gdr_mfma_bwd(d, q, k, v, g, beta, h0, d_out, d_final, dq, dk, dv, dg,
                                   dbeta, dh0, workspace, st);
    }
    GdrWs w;
    gdr_ws_layout(d, true, (char *)workspace, &w);
    GdrArgs a = gdr_args(d, q, k, v, g, beta);
    if ((rc = launch_gdr_plan(d, w, st))) return rc;
    const unsigned chunks = (unsigned)(nc * d->h), seqs = (unsigned)(S * d->h);
    const size_t smem = grads_smem();
#define BWD(DT)                                                                            \
    {                                                                                      \
        static bool attr = false;                                                          \
        if (!attr) {                                                                       \
            (void)hipFuncSetAttribute((const void *)gdr_grads<DT>,                             \
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);    \
            attr = true;                                                                   \
        }                                                                                  \
        if (chunks) gdr_prep<DT><<<chunks, 256, 0, st>>>(a, w, 1);                         \
        gdr_state_fwd<<<seqs, 256, 0, st>>>(a, w, h0, nullptr);                            \
        if (chunks) gdr_dvlocal<DT><<<chunks, 256, 0, st>>>(a, w, d_out);                  \
        gdr_state_bwd<DT><<<seqs, 256, 0, st>>>(a, w, d_out, d_final, dh0);                \
        if (chunks) gdr_grads<DT><<<chunks, 256, smem, st>>>(a, w, d_out, dq, dk, dv, dg, dbeta); \
    }
    if (d->dtype == DM_F32) {
        BWD(DM_F32)
    } else if (d->dtype == DM_BF16) {
        BWD(DM_BF16)
    } else {
        BWD(DM_F16)
    }
#undef BWD
    probe_add(DM_PROBE_GDR_CHUNK_BWD, 6);
    DM_LAUNCH_CHECK("chunk_gated_delta_rule_backward: launch");
    return DM_OK;
}

}  // extern "C"
