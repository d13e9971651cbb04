/* The causal depthwise conv1d, restated from crates/dash-ops/src/conv1d/reference.rs (TEST
 * INFRASTRUCTURE ONLY; included twice by dm_oracle.c, with R = float and R = double).
 *
 * Per sequence of L steps and channel c, with h its history (the initial state's W steps, oldest
 * first, then the inputs; zeros before those):
 *   y[t, c]   = bias[c] + sum_{j < K} weight[c, j] h[t - (K - 1) + j, c]   (reference.rs:88-106)
 *   out[t, c] = y or SiLU(y) = y sigmoid(y)                                   (reference.rs:108-114)
 * The final state is the last W' steps of h, zeros in front where it is shorter (:183-197).
 * Inputs arrive as f32 values (already the dtype's values); the arithmetic is in R. */

/* h[tau] of sequence s for tau in [-W, L): the inputs at tau >= 0, else the initial state's step
 * W + tau (reference.rs:155-171 `padded`, :173-181 `history`), zeros where there is none. */
static R FN(cv_hist)(const dmo_conv1d *p, const float *x, const float *h0, int64_t s,
                     int64_t row0, int64_t tau, int64_t c) {
    if (tau >= 0) return (R)x[(row0 + tau) * p->c + c];
    if (p->has_h0 && tau >= -p->w) return (R)h0[(s * p->w + p->w + tau) * p->c + c];
    return 0;
}

/* The pre-activation at step t: the taps summed in order j = 0 .. K - 1, then the bias
 * (reference.rs:94-105: reduce(float_add) over the taps, then add_bias). */
static R FN(cv_pre)(const dmo_conv1d *p, const float *x, const float *w, const float *bias,
                    const float *h0, int64_t s, int64_t row0, int64_t t, int64_t c) {
    R y = 0;
    for (int64_t j = 0; j < p->k; j++)
        y += (R)w[c * p->k + j] * FN(cv_hist)(p, x, h0, s, row0, t - (p->k - 1) + j, c);
    if (p->has_bias) y += (R)bias[c];
    return y;
}

static R FN(cv_sigmoid)(R y) { return 1 / (1 + EXP(-y)); }

/* The spans of the sequences: the batch rows, or the packed offsets (reference.rs:202-221). */
static void FN(cv_span)(const dmo_conv1d *p, int64_t s, int64_t *row0, int64_t *len) {
    if (p->cu) {
        *row0 = p->cu[s];
        *len = p->cu[s + 1] - p->cu[s];
    } else {
        *row0 = s * p->t;
        *len = p->t;
    }
}

/* The forward (reference.rs:223-268): out [B, T, C] (f32 values of the R result) and, with
 * has_final, the final states [S, W', C]. */
int FN(dmo_conv1d_fwd)(const dmo_conv1d *p, const float *x, const float *w, const float *bias,
                       const float *h0, float *out, float *final_state) {
    const int64_t S = p->cu ? p->nseq : p->b;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t s = 0; s < S; s++) {
        int64_t row0, L;
        FN(cv_span)(p, s, &row0, &L);
        for (int64_t t = 0; t < L; t++)
            for (int64_t c = 0; c < p->c; c++) {
                R y = FN(cv_pre)(p, x, w, bias, h0, s, row0, t, c);
                if (p->silu) y = y * FN(cv_sigmoid)(y);
                out[(row0 + t) * p->c + c] = (float)y;
            }
        if (p->has_final) {
            /* the last W' steps of the history of P = W + L steps */
            const int64_t wh = p->has_h0 ? p->w : 0, P = wh + L;
            for (int64_t i = 0; i < p->w_out; i++) {
                const int64_t tau = P - p->w_out + i - wh; /* step of the history, from x's 0 */
                for (int64_t c = 0; c < p->c; c++) {
                    R v = (tau < -wh) ? 0 : FN(cv_hist)(p, x, h0, s, row0, tau, c);
                    final_state[(s * p->w_out + i) * p->c + c] = (float)v;
                }
            }
        }
    }
    return 0;
}

/* The backward (reference.rs:270-506), given the output's gradient go [B, T, C] and, with
 * has_final, the final states' gradient gfin [S, W', C]: gx [B, T, C], gw [C, K] and gb [C]
 * (sums over every step of every sequence, sequence by sequence), gh0 [S, W, C] with has_h0. */
int FN(dmo_conv1d_bwd)(const dmo_conv1d *p, const float *x, const float *w, const float *bias,
                       const float *h0, const float *go, const float *gfin, float *gx, float *gw,
                       float *gb, float *gh0) {
    const int64_t S = p->cu ? p->nseq : p->b, K = p->k, C = p->c;
    const int64_t wh = p->has_h0 ? p->w : 0;
    R *sw = (R *)calloc((size_t)(S * C * K), sizeof(R)); /* per sequence, then summed in order */
    R *sb = (R *)calloc((size_t)(S * C), sizeof(R));
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t s = 0; s < S; s++) {
        int64_t row0, L;
        FN(cv_span)(p, s, &row0, &L);
        R *gy = (R *)malloc((size_t)((L > 0 ? L : 1) * C) * sizeof(R));
        /* the pre-activation's gradient: go SiLU'(y), SiLU'(y) = s (1 + y (1 - s)) (:117-134) */
        for (int64_t t = 0; t < L; t++)
            for (int64_t c = 0; c < C; c++) {
                R g = (R)go[(row0 + t) * C + c];
                if (p->silu) {
                    const R y = FN(cv_pre)(p, x, w, bias, h0, s, row0, t, c);
                    const R sg = FN(cv_sigmoid)(y);
                    g = g * (sg * (y * (1 - sg) + 1));
                }
                gy[t * C + c] = g;
            }
        for (int64_t c = 0; c < C; c++) {
            /* the padded steps' gradient: padded step q feeds outputs q - (K - 1) .. q through
             * taps K - 1 .. 0 (:296-316), summed over the taps in order */
            for (int64_t q = 0; q < L + K - 1; q++) {
                R g = 0;
                for (int64_t j = 0; j < K; j++) {
                    const int64_t t = q - j;
                    if (t >= 0 && t < L) g += (R)w[c * K + j] * gy[t * C + c];
                }
                if (q >= K - 1)
                    gx[(row0 + q - (K - 1)) * C + c] = (float)g;
                else if (p->has_h0) /* the initial state's last K - 1 steps (:318-325) */
                    gh0[(s * p->w + p->w - (K - 1) + q) * C + c] = (float)g;
            }
            if (p->has_h0)
                for (int64_t i = 0; i < p->w - (K - 1); i++) gh0[(s * p->w + i) * C + c] = 0;
            if (p->has_h0 && L == 0)
                for (int64_t i = 0; i < p->w; i++) gh0[(s * p->w + i) * C + c] = 0;
            /* the weight's and the bias's sums over the steps (:326-340) */
            for (int64_t j = 0; j < K; j++) {
                R a = 0;
                for (int64_t t = 0; t < L; t++)
                    a += gy[t * C + c] * FN(cv_hist)(p, x, h0, s, row0, t - (K - 1) + j, c);
                sw[(s * C + c) * K + j] = a;
            }
            R a = 0;
            for (int64_t t = 0; t < L; t++) a += gy[t * C + c];
            sb[s * C + c] = a;
            /* the final states' gradient onto the history's last W' steps (:342-373) */
            if (p->has_final) {
                const int64_t P = wh + L;
                for (int64_t i = 0; i < p->w_out; i++) {
                    const int64_t hstep = P - p->w_out + i; /* history step, from 0 */
                    if (hstep < 0) continue;
                    const R g = (R)gfin[(s * p->w_out + i) * C + c];
                    if (hstep >= wh) {
                        float *d = &gx[(row0 + hstep - wh) * C + c];
                        *d = (float)((R)*d + g);
                    } else {
                        float *d = &gh0[(s * p->w + hstep) * C + c];
                        *d = (float)((R)*d + g);
                    }
                }
            }
        }
        free(gy);
    }
    for (int64_t c = 0; c < C; c++) {
        for (int64_t j = 0; j < K; j++) {
            R a = 0;
            for (int64_t s = 0; s < S; s++) a += sw[(s * C + c) * K + j];
            gw[c * K + j] = (float)a;
        }
        if (p->has_bias) {
            R a = 0;
            for (int64_t s = 0; s < S; s++) a += sb[s * C + c];
            gb[c] = (float)a;
        }
    }
    free(sw);
    free(sb);
    return 0;
}

/* One decoding step (reference.rs:484-520): x [B, C], state [B, W, C] to out [B, C] and the next
 * state [B, W, C]: the state's last K - 1 steps and the token through the taps, summed in order;
 * the state without its oldest step, then the token. */
int FN(dmo_conv1d_update)(int64_t b, int64_t c, int64_t k, int64_t w, int32_t has_bias,
                          int32_t silu, const float *x, const float *wt, const float *bias,
                          const float *state, float *out, float *next) {
    for (int64_t bi = 0; bi < b; bi++)
        for (int64_t ci = 0; ci < c; ci++) {
            R y = 0;
            for (int64_t j = 0; j < k; j++) {
                const R v = j < k - 1 ? (R)state[(bi * w + w - (k - 1) + j) * c + ci]
                                      : (R)x[bi * c + ci];
                y += v * (R)wt[ci * k + j];
            }
            if (has_bias) y += (R)bias[ci];
            if (silu) y = y * FN(cv_sigmoid)(y);
            out[bi * c + ci] = (float)y;
            for (int64_t i = 0; i < w; i++)
                next[(bi * w + i) * c + ci] =
                    i + 1 < w ? state[(bi * w + i + 1) * c + ci] : x[bi * c + ci];
        }
    return 0;
}
