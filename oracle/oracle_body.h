/* Body of the CPU oracle, included once per precision by dm_oracle.c with
 *   R      the arithmetic type (float: the reference's own precision; double: a tighter checker)
 *   FN(x)  the function name with the precision's suffix.
 *
 * TEST INFRASTRUCTURE ONLY. This is a restatement of dash-ops' reference implementations, used
 * by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker. The product
 * path (dashmag_amd, libdashmi.so) never calls it.
 *
 * Layouts are the contract's (crates/dash-contract/src/lib.rs:38-60): [B, T, H, D] row-major,
 * states [S, H, Dk, Dv], all given and returned as f32 arrays whatever R is.
 */

/* ------------------------------------------------------------------------------------------ */
/* Attention: crates/dash-ops/src/attention/reference.rs                                      */
/* ------------------------------------------------------------------------------------------ */

/* Forward for one (batch, query head, query row): reference.rs:305-348 (forward_hidden), the
 * scores materialised over the row, -inf where hidden, max replaced by 0 for an empty row, the
 * probabilities divided by the sum (1 where the sum is 0), lse = max + log(sum). */
static void FN(attn_row_fwd)(const dmo_attention *a, const float *q, const float *k,
                             const float *v, float *o, float *lse, int64_t b, int64_t h,
                             int64_t i, R *scores) {
    const int64_t tk = a->tk, d = a->d, hkv = a->hkv, group = a->hq / a->hkv;
    const int64_t kh = h / group;
    const float *qi = q + ((b * a->tq + i) * a->hq + h) * d;
    R mx = -INFINITY;
    for (int64_t j = 0; j < tk; j++) {
        if (!dmo_attention_visible(a, b, i, j)) {
            scores[j] = -INFINITY;
            continue;
        }
        const float *kj = k + ((b * tk + j) * hkv + kh) * d;
        R s = 0;
        for (int64_t x = 0; x < d; x++) s += (R)qi[x] * (R)kj[x];
        s = s * (R)a->scale;
        scores[j] = s;
        if (s > mx) mx = s;
    }
    if (mx == -INFINITY) mx = 0;
    R sum = 0;
    for (int64_t j = 0; j < tk; j++) {
        scores[j] = EXP(scores[j] - mx);
        sum += scores[j];
    }
    R div = sum == 0 ? (R)1 : sum;
    float *oi = o + ((b * a->tq + i) * a->hq + h) * d;
    for (int64_t x = 0; x < d; x++) {
        R acc = 0;
        for (int64_t j = 0; j < tk; j++) {
            if (scores[j] == 0) continue;
            acc += (scores[j] / div) * (R)v[((b * tk + j) * hkv + kh) * d + x];
        }
        oi[x] = (float)acc;
    }
    lse[(b * a->tq + i) * a->hq + h] = (float)(mx + LOG(sum));
}

int FN(dmo_attention_fwd)(const dmo_attention *a, const float *q, const float *k,
                          const float *v, float *o, float *lse) {
    const int64_t rows = a->b * a->hq * a->tq;
    if (a->tk == 0) {
        for (int64_t r = 0; r < rows; r++) lse[r] = -INFINITY;
        memset(o, 0, sizeof(float) * rows * a->d);
        return 0;
    }
#pragma omp parallel
    {
        R *scores = (R *)malloc(sizeof(R) * a->tk);
#pragma omp for schedule(dynamic, 4)
        for (int64_t r = 0; r < rows; r++) {
            int64_t i = r % a->tq, h = (r / a->tq) % a->hq, b = r / (a->tq * a->hq);
            FN(attn_row_fwd)(a, q, k, v, o, lse, b, h, i, scores);
        }
        free(scores);
    }
    return 0;
}

/* Backward: reference.rs:352-431. P = exp(S - lse) with lse -inf read as +inf (P = 0 for an
 * empty row), dV = P^T dO, dP = dO V^T, delta = rowsum(dO * O), dS = P (dP - delta),
 * dQ = scale dS K, dK = scale dS^T Q, the key-value gradients summed over each group. The query
 * gradient runs per query row and the key-value gradients per key row, so that every output
 * element is one sequential sum. */
static R FN(attn_prob)(const dmo_attention *a, const float *q, const float *k, const float *lse,
                       int64_t b, int64_t h, int64_t i, int64_t j) {
    if (!dmo_attention_visible(a, b, i, j)) return 0;
    const int64_t d = a->d, group = a->hq / a->hkv, kh = h / group;
    const float *qi = q + ((b * a->tq + i) * a->hq + h) * d;
    const float *kj = k + ((b * a->tk + j) * a->hkv + kh) * d;
    R s = 0;
    for (int64_t x = 0; x < d; x++) s += (R)qi[x] * (R)kj[x];
    s = s * (R)a->scale;
    R l = lse[(b * a->tq + i) * a->hq + h];
    if (l == -INFINITY) l = INFINITY;
    return EXP(s - l);
}

static R FN(attn_dprob)(const dmo_attention *a, const float *v, const float *d_o, int64_t b,
                        int64_t h, int64_t i, int64_t j) {
    const int64_t d = a->d, group = a->hq / a->hkv, kh = h / group;
    const float *gi = d_o + ((b * a->tq + i) * a->hq + h) * d;
    const float *vj = v + ((b * a->tk + j) * a->hkv + kh) * d;
    R s = 0;
    for (int64_t x = 0; x < d; x++) s += (R)gi[x] * (R)vj[x];
    return s;
}

int FN(dmo_attention_bwd)(const dmo_attention *a, const float *q, const float *k,
                          const float *v, const float *o, const float *lse, const float *d_o,
                          float *dq, float *dk, float *dv) {
    const int64_t tq = a->tq, tk = a->tk, hq = a->hq, hkv = a->hkv, d = a->d;
    const int64_t group = hq / hkv;
    const int64_t qrows = a->b * hq * tq, krows = a->b * hkv * tk;
    memset(dq, 0, sizeof(float) * qrows * d);
    memset(dk, 0, sizeof(float) * krows * d);
    memset(dv, 0, sizeof(float) * krows * d);
    if (tk == 0 || tq == 0) return 0;
    R *delta = (R *)malloc(sizeof(R) * qrows);
#pragma omp parallel for
    for (int64_t r = 0; r < qrows; r++) {
        const float *gi = d_o + r * d, *oi = o + r * d;
        R s = 0;
        for (int64_t x = 0; x < d; x++) s += (R)gi[x] * (R)oi[x];
        delta[r] = s;
    }
#pragma omp parallel
    {
        R *acc = (R *)malloc(sizeof(R) * d * 2);
#pragma omp for schedule(dynamic, 4)
        for (int64_t r = 0; r < qrows; r++) {
            /* r indexes [B, Tq, Hq] rows */
            int64_t h = r % hq, i = (r / hq) % tq, b = r / (hq * tq);
            int64_t kh = h / group;
            for (int64_t x = 0; x < d; x++) acc[x] = 0;
            for (int64_t j = 0; j < tk; j++) {
                R p = FN(attn_prob)(a, q, k, lse, b, h, i, j);
                if (p == 0) continue;
                R ds = p * (FN(attn_dprob)(a, v, d_o, b, h, i, j) - delta[r]);
                const float *kj = k + ((b * tk + j) * hkv + kh) * d;
                for (int64_t x = 0; x < d; x++) acc[x] += ds * (R)kj[x];
            }
            for (int64_t x = 0; x < d; x++) dq[r * d + x] = (float)(acc[x] * (R)a->scale);
        }
#pragma omp for schedule(dynamic, 4)
        for (int64_t r = 0; r < krows; r++) {
            /* r indexes [B, Tk, Hkv] rows */
            int64_t kh = r % hkv, j = (r / hkv) % tk, b = r / (hkv * tk);
            R *ak = acc, *av = acc + d;
            for (int64_t x = 0; x < 2 * d; x++) acc[x] = 0;
            for (int64_t h = kh * group; h < (kh + 1) * group; h++) {
                for (int64_t i = 0; i < tq; i++) {
                    R p = FN(attn_prob)(a, q, k, lse, b, h, i, j);
                    if (p == 0) continue;
                    int64_t qr = (b * tq + i) * hq + h;
                    R ds = p * (FN(attn_dprob)(a, v, d_o, b, h, i, j) - delta[qr]);
                    const float *qi = q + qr * d, *gi = d_o + qr * d;
                    for (int64_t x = 0; x < d; x++) {
                        av[x] += p * (R)gi[x];
                        ak[x] += ds * (R)qi[x];
                    }
                }
            }
            for (int64_t x = 0; x < d; x++) {
                dk[r * d + x] = (float)(ak[x] * (R)a->scale);
                dv[r * d + x] = (float)av[x];
            }
        }
        free(acc);
    }
    free(delta);
    return 0;
}

/* Decoding: reference.rs:433-467. One query per sequence, [B, Hq, D], against [B, S, Hkv, D];
 * sequence b sees keys max(0, len - 1 - left) <= j < len, len = lengths[b] (S without lengths),
 * the query after its last key. */
int FN(dmo_attention_decode)(int64_t b, int64_t s, int64_t hq, int64_t hkv, int64_t d,
                             const float *q, const float *k, const float *v,
                             const int64_t *lengths, int64_t left, float scale, float *o) {
    const int64_t group = hq / hkv;
#pragma omp parallel
    {
        R *scores = (R *)malloc(sizeof(R) * (s > 0 ? s : 1));
#pragma omp for schedule(dynamic, 1)
        for (int64_t r = 0; r < b * hq; r++) {
            int64_t bi = r / hq, h = r % hq, kh = h / group;
            int64_t len = lengths ? lengths[bi] : s;
            int64_t lo = 0;
            if (left >= 0 && left < s + 1) lo = len - 1 - left;
            if (lo < 0) lo = 0;
            if (len > s) len = s;
            const float *qi = q + r * d;
            R mx = -INFINITY;
            for (int64_t j = 0; j < s; j++) {
                if (j < lo || j >= len) {
                    scores[j] = -INFINITY;
                    continue;
                }
                const float *kj = k + ((bi * s + j) * hkv + kh) * d;
                R acc = 0;
                for (int64_t x = 0; x < d; x++) acc += (R)qi[x] * (R)kj[x];
                scores[j] = acc * (R)scale;
                if (scores[j] > mx) mx = scores[j];
            }
            if (mx == -INFINITY) mx = 0;
            R sum = 0;
            for (int64_t j = 0; j < s; j++) {
                scores[j] = EXP(scores[j] - mx);
                sum += scores[j];
            }
            R div = sum == 0 ? (R)1 : sum;
            for (int64_t x = 0; x < d; x++) {
                R acc = 0;
                for (int64_t j = 0; j < s; j++) {
                    if (scores[j] == 0) continue;
                    acc += (scores[j] / div) * (R)v[((bi * s + j) * hkv + kh) * d + x];
                }
                o[r * d + x] = (float)acc;
            }
        }
        free(scores);
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* Gated delta rule, chunked: crates/dash-ops/src/gated_delta/chunk/reference.rs              */
/* ------------------------------------------------------------------------------------------ */

#define C DMO_CHUNK

/* c[m][n] (+)= a[m][k] b[k][n] with element strides given as (row, col) pairs, so that any
 * operand can be read transposed. */
static void FN(mm)(int64_t m, int64_t n, int64_t kk, const R *a, int64_t ar, int64_t ac,
                   const R *b, int64_t br, int64_t bc, R *c, int accumulate) {
    for (int64_t i = 0; i < m; i++)
        for (int64_t j = 0; j < n; j++) {
            R s = 0;
            for (int64_t x = 0; x < kk; x++) s += a[i * ar + x * ac] * b[x * br + j * bc];
            c[i * n + j] = accumulate ? c[i * n + j] + s : s;
        }
}

/* Per-chunk quantities of one (sequence, head): chunk/reference.rs notation :11-18 and
 * `intra` :429-479. */
typedef struct {
    R q[C * DMO_DMAX], k[C * DMO_DMAX], v[C * DMO_DMAX];
    R g[C], beta[C], G[C], gamma[C], lam[C], gl;
    R decay[C * C], A[C * C], T[C * C];
    R W[C * DMO_DMAX], U[C * DMO_DMAX], kt[C * DMO_DMAX];
} FN(chunk_t);

/* Loads chunk c of tokens [t0, t0 + len) of head h, zero-padded (chunk4/chunk3 :192-229),
 * l2-normalised if asked (l2norm :234) and the queries scaled (prepare :284-311). */
static void FN(chunk_load)(const dmo_gdr *p, const float *q, const float *k, const float *v,
                           const float *g, const float *beta, int64_t t0, int64_t len,
                           int64_t h, int64_t c, FN(chunk_t) * ch) {
    const int64_t H = p->h, dk = p->dk, dv = p->dv;
    memset(ch->q, 0, sizeof(ch->q));
    memset(ch->k, 0, sizeof(ch->k));
    memset(ch->v, 0, sizeof(ch->v));
    for (int64_t i = 0; i < C; i++) {
        int64_t t = c * C + i;
        if (t >= len) {
            ch->g[i] = 0;
            ch->beta[i] = 0;
            continue;
        }
        int64_t tok = t0 + t;
        const float *qt = q + (tok * H + h) * dk, *kt = k + (tok * H + h) * dk;
        R qs = 0, ks = 0;
        for (int64_t x = 0; x < dk; x++) {
            qs += (R)qt[x] * (R)qt[x];
            ks += (R)kt[x] * (R)kt[x];
        }
        R qi = 1, ki = 1;
        if (p->qk_l2norm) {
            qi = (R)1 / SQRT(qs + (R)DMO_L2NORM_EPS);
            ki = (R)1 / SQRT(ks + (R)DMO_L2NORM_EPS);
        }
        for (int64_t x = 0; x < dk; x++) {
            R qn = p->qk_l2norm ? (R)qt[x] * qi : (R)qt[x];
            ch->q[i * dk + x] = qn * (R)p->scale;
            ch->k[i * dk + x] = p->qk_l2norm ? (R)kt[x] * ki : (R)kt[x];
        }
        for (int64_t x = 0; x < dv; x++) ch->v[i * dv + x] = (R)v[(tok * H + h) * dv + x];
        ch->g[i] = (R)g[tok * H + h];
        ch->beta[i] = (R)beta[tok * H + h];
    }
}

/* `intra` (:429-479) with `unit_lower_inverse` (:330-345), `lam` and `g_last` (:450-466). */
static void FN(chunk_intra)(const dmo_gdr *p, FN(chunk_t) * ch) {
    const int64_t dk = p->dk, dv = p->dv;
    R acc = 0;
    for (int64_t i = 0; i < C; i++) {
        acc += ch->g[i];
        ch->G[i] = acc;
        ch->gamma[i] = EXP(acc);
    }
    for (int64_t i = 0; i < C; i++) ch->lam[i] = EXP(ch->G[C - 1] - ch->G[i]);
    ch->gl = EXP(ch->G[C - 1]);
    for (int64_t i = 0; i < C; i++)
        for (int64_t j = 0; j < C; j++) {
            /* masked before the exponential, as the reference does */
            R diff = i >= j ? ch->G[i] - ch->G[j] : 0;
            ch->decay[i * C + j] = i >= j ? EXP(diff) : 0;
        }
    for (int64_t i = 0; i < C; i++)
        for (int64_t j = 0; j < C; j++) {
            R s = 0;
            if (i > j) {
                for (int64_t x = 0; x < dk; x++)
                    s += ch->k[i * dk + x] * ch->beta[i] * ch->k[j * dk + x];
                s *= ch->decay[i * C + j];
            }
            ch->A[i * C + j] = s;
        }
    /* (I + A)^-1 by forward substitution: m = -A; row i += row i . m[:i, :i]; then + I. */
    R *m = ch->T;
    for (int64_t x = 0; x < C * C; x++) m[x] = -ch->A[x];
    for (int64_t i = 1; i < C; i++) {
        R row[C];
        for (int64_t j = 0; j < i; j++) {
            R s = 0;
            for (int64_t x = 0; x < i; x++) s += m[i * C + x] * m[x * C + j];
            row[j] = m[i * C + j] + s;
        }
        for (int64_t j = 0; j < i; j++) m[i * C + j] = row[j];
    }
    for (int64_t i = 0; i < C; i++) m[i * C + i] += 1;
    /* W = T (beta gamma K), U = T (beta V), kt = lam K */
    R *tmp = (R *)malloc(sizeof(R) * C * DMO_DMAX);
    for (int64_t i = 0; i < C; i++)
        for (int64_t x = 0; x < dk; x++)
            tmp[i * dk + x] = ch->k[i * dk + x] * ch->beta[i] * ch->gamma[i];
    FN(mm)(C, dk, C, ch->T, C, 1, tmp, dk, 1, ch->W, 0);
    for (int64_t i = 0; i < C; i++)
        for (int64_t x = 0; x < dv; x++) tmp[i * dv + x] = ch->v[i * dv + x] * ch->beta[i];
    FN(mm)(C, dv, C, ch->T, C, 1, tmp, dv, 1, ch->U, 0);
    for (int64_t i = 0; i < C; i++)
        for (int64_t x = 0; x < dk; x++) ch->kt[i * dk + x] = ch->k[i * dk + x] * ch->lam[i];
    free(tmp);
}

/* One sequence and head forward (forward :481-509, state_forward :348-372): out rows
 * [t0, t0 + len), final state into `state` (which holds the initial state on entry). */
static void FN(gdr_forward_one)(const dmo_gdr *p, const float *q, const float *k,
                                const float *v, const float *g, const float *beta, int64_t t0,
                                int64_t len, int64_t h, R *state, float *out) {
    const int64_t dk = p->dk, dv = p->dv, n = (len + C - 1) / C, H = p->h;
    FN(chunk_t) *ch = (FN(chunk_t) *)malloc(sizeof(FN(chunk_t)));
    R *vn = (R *)malloc(sizeof(R) * C * dv);
    R *o = (R *)malloc(sizeof(R) * C * dv);
    R *qg = (R *)malloc(sizeof(R) * C * dk);
    R *attn = (R *)malloc(sizeof(R) * C * C);
    for (int64_t c = 0; c < n; c++) {
        FN(chunk_load)(p, q, k, v, g, beta, t0, len, h, c, ch);
        FN(chunk_intra)(p, ch);
        /* V' = U - W S */
        FN(mm)(C, dv, dk, ch->W, dk, 1, state, dv, 1, vn, 0);
        for (int64_t x = 0; x < C * dv; x++) vn[x] = ch->U[x] - vn[x];
        /* O = (gamma Q) S + ((Q K^T) decay) V' */
        for (int64_t i = 0; i < C; i++)
            for (int64_t x = 0; x < dk; x++) qg[i * dk + x] = ch->q[i * dk + x] * ch->gamma[i];
        FN(mm)(C, dv, dk, qg, dk, 1, state, dv, 1, o, 0);
        FN(mm)(C, C, dk, ch->q, dk, 1, ch->k, 1, dk, attn, 0);
        for (int64_t x = 0; x < C * C; x++) attn[x] *= ch->decay[x];
        FN(mm)(C, dv, C, attn, C, 1, vn, dv, 1, o, 1);
        for (int64_t i = 0; i < C && c * C + i < len; i++)
            for (int64_t x = 0; x < dv; x++)
                out[((t0 + c * C + i) * H + h) * dv + x] = (float)o[i * dv + x];
        /* S <- exp(G_last) S + (lam K)^T V' */
        for (int64_t x = 0; x < dk * dv; x++) state[x] *= ch->gl;
        FN(mm)(dk, dv, C, ch->kt, 1, dk, vn, dv, 1, state, 1);
    }
    free(ch);
    free(vn);
    free(o);
    free(qg);
    free(attn);
}

/* The sequences of a call: packed (`cu` [S + 1] over one batch row) or one per batch row. */
static int64_t FN(gdr_spans)(const dmo_gdr *p, int64_t s, int64_t *t0, int64_t *len) {
    if (p->cu) {
        *t0 = p->cu[s];
        *len = p->cu[s + 1] - p->cu[s];
    } else {
        *t0 = s * p->t;
        *len = p->t;
    }
    return 0;
}

int FN(dmo_gdr_chunk_fwd)(const dmo_gdr *p, const float *q, const float *k, const float *v,
                          const float *g, const float *beta, const float *h0, float *out,
                          float *final_state) {
    const int64_t S = p->cu ? p->nseq : p->b, H = p->h, dk = p->dk, dv = p->dv;
    if (dk > DMO_DMAX || dv > DMO_DMAX) return -1;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t r = 0; r < S * H; r++) {
        int64_t s = r / H, h = r % H, t0, len;
        FN(gdr_spans)(p, s, &t0, &len);
        R *state = (R *)malloc(sizeof(R) * dk * dv);
        for (int64_t x = 0; x < dk * dv; x++) state[x] = h0 ? (R)h0[r * dk * dv + x] : 0;
        FN(gdr_forward_one)(p, q, k, v, g, beta, t0, len, h, state, out);
        for (int64_t x = 0; x < dk * dv; x++) final_state[r * dk * dv + x] = (float)state[x];
        free(state);
    }
    return 0;
}

/* The backward of one sequence and head, written out as chunk/reference.rs:519-695 does, with
 * the state's gradient passed back chunk to chunk (state_backward :382-427). */
static void FN(gdr_backward_one)(const dmo_gdr *p, const float *q, const float *k,
                                 const float *v, const float *g, const float *beta,
                                 const float *h0, const float *d_out, const float *d_final,
                                 int64_t t0, int64_t len, int64_t h, int64_t r, float *dq_out,
                                 float *dk_out, float *dv_out, float *dg_out, float *dbeta_out,
                                 float *dh0_out) {
    const int64_t dk = p->dk, dv = p->dv, n = (len + C - 1) / C, H = p->h;
    const int64_t SS = dk * dv;
    FN(chunk_t) *chs = (FN(chunk_t) *)malloc(sizeof(FN(chunk_t)) * n);
    R *states = (R *)malloc(sizeof(R) * SS * (n + 1));
    R *vns = (R *)malloc(sizeof(R) * C * dv * n);
    R *dos = (R *)calloc(C * dv * n, sizeof(R));
    R *ds_next = (R *)malloc(sizeof(R) * SS * n);
    R *dvns = (R *)malloc(sizeof(R) * C * dv * n);
    /* forward recompute */
    for (int64_t x = 0; x < SS; x++) states[x] = h0 ? (R)h0[r * SS + x] : 0;
    for (int64_t c = 0; c < n; c++) {
        FN(chunk_t) *ch = &chs[c];
        FN(chunk_load)(p, q, k, v, g, beta, t0, len, h, c, ch);
        FN(chunk_intra)(p, ch);
        R *s = states + c * SS, *sn = states + (c + 1) * SS, *vn = vns + c * C * dv;
        FN(mm)(C, dv, dk, ch->W, dk, 1, s, dv, 1, vn, 0);
        for (int64_t x = 0; x < C * dv; x++) vn[x] = ch->U[x] - vn[x];
        for (int64_t x = 0; x < SS; x++) sn[x] = s[x] * ch->gl;
        FN(mm)(dk, dv, C, ch->kt, 1, dk, vn, dv, 1, sn, 1);
        for (int64_t i = 0; i < C && c * C + i < len; i++)
            for (int64_t x = 0; x < dv; x++)
                dos[(c * C + i) * dv + x] = (R)d_out[((t0 + c * C + i) * H + h) * dv + x];
    }
    /* state backward */
    R *ds = (R *)malloc(sizeof(R) * SS);
    R *tmp = (R *)malloc(sizeof(R) * SS);
    R *qg = (R *)malloc(sizeof(R) * C * DMO_DMAX);
    R *attn = (R *)malloc(sizeof(R) * C * C);
    R *dvl = (R *)malloc(sizeof(R) * C * dv);
    for (int64_t x = 0; x < SS; x++) ds[x] = d_final ? (R)d_final[r * SS + x] : 0;
    for (int64_t c = n - 1; c >= 0; c--) {
        FN(chunk_t) *ch = &chs[c];
        R *d_o = dos + c * C * dv, *dvn = dvns + c * C * dv;
        memcpy(ds_next + c * SS, ds, sizeof(R) * SS);
        /* dv_local = attn^T dO */
        FN(mm)(C, C, dk, ch->q, dk, 1, ch->k, 1, dk, attn, 0);
        for (int64_t x = 0; x < C * C; x++) attn[x] *= ch->decay[x];
        FN(mm)(C, dv, C, attn, 1, C, d_o, dv, 1, dvl, 0);
        /* dV'_c = kt_c dS_{c+1} + dv_local_c */
        FN(mm)(C, dv, dk, ch->kt, dk, 1, ds, dv, 1, dvn, 0);
        for (int64_t x = 0; x < C * dv; x++) dvn[x] += dvl[x];
        /* dS_c = exp(G_last) dS_{c+1} + qg^T dO - W^T dV' */
        for (int64_t i = 0; i < C; i++)
            for (int64_t x = 0; x < dk; x++) qg[i * dk + x] = ch->q[i * dk + x] * ch->gamma[i];
        FN(mm)(dk, dv, C, qg, 1, dk, d_o, dv, 1, tmp, 0);
        for (int64_t x = 0; x < SS; x++) ds[x] = ds[x] * ch->gl + tmp[x];
        FN(mm)(dk, dv, C, ch->W, 1, dk, dvn, dv, 1, tmp, 0);
        for (int64_t x = 0; x < SS; x++) ds[x] -= tmp[x];
    }
    if (dh0_out)
        for (int64_t x = 0; x < SS; x++) dh0_out[r * SS + x] = (float)ds[x];

    /* per-chunk gradients */
    R *dqc = (R *)malloc(sizeof(R) * C * DMO_DMAX), *dkc = (R *)malloc(sizeof(R) * C * DMO_DMAX);
    R *dvc = (R *)malloc(sizeof(R) * C * DMO_DMAX), *d_qg = (R *)malloc(sizeof(R) * C * DMO_DMAX);
    R *dkt = (R *)malloc(sizeof(R) * C * DMO_DMAX), *dw = (R *)malloc(sizeof(R) * C * DMO_DMAX);
    R *dkbg = (R *)malloc(sizeof(R) * C * DMO_DMAX), *dvb = (R *)malloc(sizeof(R) * C * DMO_DMAX);
    R *dkbeta = (R *)malloc(sizeof(R) * C * DMO_DMAX), *vb = (R *)malloc(sizeof(R) * C * DMO_DMAX);
    R *kbg = (R *)malloc(sizeof(R) * C * DMO_DMAX);
    R *dattn = (R *)malloc(sizeof(R) * C * C), *dT = (R *)malloc(sizeof(R) * C * C);
    R *m1 = (R *)malloc(sizeof(R) * C * C), *dA = (R *)malloc(sizeof(R) * C * C);
    R d_gamma[C], d_g[C], d_beta[C];
    for (int64_t c = 0; c < n; c++) {
        FN(chunk_t) *ch = &chs[c];
        R *S = states + c * SS, *dsn = ds_next + c * SS, *vn = vns + c * C * dv;
        R *d_o = dos + c * C * dv, *dvn = dvns + c * C * dv;
        FN(mm)(C, C, dk, ch->q, dk, 1, ch->k, 1, dk, attn, 0);
        for (int64_t x = 0; x < C * C; x++) attn[x] *= ch->decay[x];
        /* O = (gamma Q) S + P V' */
        FN(mm)(C, dk, dv, d_o, dv, 1, S, 1, dv, d_qg, 0);
        for (int64_t i = 0; i < C; i++) {
            R s = 0;
            for (int64_t x = 0; x < dk; x++) {
                dqc[i * dk + x] = d_qg[i * dk + x] * ch->gamma[i];
                s += d_qg[i * dk + x] * ch->q[i * dk + x];
            }
            d_gamma[i] = s;
        }
        FN(mm)(C, C, dv, d_o, dv, 1, vn, 1, dv, dattn, 0);
        for (int64_t i = 0; i < C; i++)
            for (int64_t j = 0; j < C; j++)
                if (j > i) dattn[i * C + j] = 0;
        /* d_attn_e = d_attn decay */
        for (int64_t x = 0; x < C * C; x++) m1[x] = dattn[x] * ch->decay[x];
        FN(mm)(C, dk, C, m1, C, 1, ch->k, dk, 1, dqc, 1);
        FN(mm)(C, dk, C, m1, 1, C, ch->q, dk, 1, dkc, 0);
        for (int64_t x = 0; x < C * C; x++) m1[x] = dattn[x] * attn[x];
        for (int64_t i = 0; i < C; i++) {
            R rs = 0, cs = 0;
            for (int64_t j = 0; j < C; j++) {
                rs += m1[i * C + j];
                cs += m1[j * C + i];
            }
            d_g[i] = rs - cs;
        }
        /* S_next = exp(G_last) S + (lam K)^T V' */
        FN(mm)(C, dk, dv, vn, dv, 1, dsn, 1, dv, dkt, 0);
        R lam_sum = 0;
        for (int64_t i = 0; i < C; i++) {
            R s = 0;
            for (int64_t x = 0; x < dk; x++) {
                dkc[i * dk + x] += dkt[i * dk + x] * ch->lam[i];
                s += dkt[i * dk + x] * ch->k[i * dk + x];
            }
            R lam_dlam = s * ch->lam[i];
            d_g[i] -= lam_dlam;
            lam_sum += lam_dlam;
        }
        R s_ds = 0;
        for (int64_t x = 0; x < SS; x++) s_ds += S[x] * dsn[x];
        d_g[C - 1] += lam_sum + s_ds * ch->gl;
        /* V' = U - W S */
        FN(mm)(C, dk, dv, dvn, dv, 1, S, 1, dv, dw, 0);
        for (int64_t x = 0; x < C * dk; x++) dw[x] = -dw[x];
        /* W = T (beta gamma K), U = T (beta V) */
        for (int64_t i = 0; i < C; i++) {
            for (int64_t x = 0; x < dv; x++) vb[i * dv + x] = ch->v[i * dv + x] * ch->beta[i];
            for (int64_t x = 0; x < dk; x++)
                kbg[i * dk + x] = ch->k[i * dk + x] * ch->beta[i] * ch->gamma[i];
        }
        FN(mm)(C, C, dv, dvn, dv, 1, vb, 1, dv, dT, 0);
        FN(mm)(C, C, dk, dw, dk, 1, kbg, 1, dk, dT, 1);
        FN(mm)(C, dv, C, ch->T, 1, C, dvn, dv, 1, dvb, 0);
        FN(mm)(C, dk, C, ch->T, 1, C, dw, dk, 1, dkbg, 0);
        for (int64_t i = 0; i < C; i++) {
            R s1 = 0, s2 = 0, s3 = 0;
            for (int64_t x = 0; x < dv; x++) {
                dvc[i * dv + x] = dvb[i * dv + x] * ch->beta[i];
                s1 += dvb[i * dv + x] * ch->v[i * dv + x];
            }
            for (int64_t x = 0; x < dk; x++) {
                s2 += dkbg[i * dk + x] * ch->k[i * dk + x] * ch->gamma[i];
                dkc[i * dk + x] += dkbg[i * dk + x] * ch->beta[i] * ch->gamma[i];
                s3 += dkbg[i * dk + x] * ch->k[i * dk + x] * ch->beta[i];
            }
            d_beta[i] = s1 + s2;
            d_gamma[i] += s3;
            d_g[i] += d_gamma[i] * ch->gamma[i];
        }
        /* dA = -(T^T dT T^T), strictly lower */
        FN(mm)(C, C, C, ch->T, 1, C, dT, C, 1, m1, 0);
        FN(mm)(C, C, C, m1, C, 1, ch->T, 1, C, dA, 0);
        for (int64_t i = 0; i < C; i++)
            for (int64_t j = 0; j < C; j++) dA[i * C + j] = i > j ? -dA[i * C + j] : 0;
        /* A = (beta K K^T) decay, strictly lower */
        for (int64_t i = 0; i < C; i++)
            for (int64_t j = 0; j < C; j++)
                m1[i * C + j] = i > j ? dA[i * C + j] * ch->decay[i * C + j] : 0;
        FN(mm)(C, dk, C, m1, C, 1, ch->k, dk, 1, dkbeta, 0);
        for (int64_t i = 0; i < C; i++) {
            R s = 0;
            for (int64_t x = 0; x < dk; x++) {
                dkc[i * dk + x] += dkbeta[i * dk + x] * ch->beta[i];
                s += dkbeta[i * dk + x] * ch->k[i * dk + x];
            }
            d_beta[i] += s;
        }
        for (int64_t i = 0; i < C; i++)
            for (int64_t x = 0; x < dk; x++) kbg[i * dk + x] = ch->k[i * dk + x] * ch->beta[i];
        FN(mm)(C, dk, C, m1, 1, C, kbg, dk, 1, dkc, 1);
        for (int64_t x = 0; x < C * C; x++) m1[x] = dA[x] * ch->A[x];
        for (int64_t i = 0; i < C; i++) {
            R rs = 0, cs = 0;
            for (int64_t j = 0; j < C; j++) {
                rs += m1[i * C + j];
                cs += m1[j * C + i];
            }
            d_g[i] += rs - cs;
        }
        /* G = cumsum(g): dg is the reverse cumulative sum of dG */
        R tail = 0;
        R dgc[C];
        for (int64_t i = C - 1; i >= 0; i--) {
            tail += d_g[i];
            dgc[i] = tail;
        }
        /* write back, undoing the scale and the l2 normalisation (l2norm_backward :246) */
        for (int64_t i = 0; i < C && c * C + i < len; i++) {
            int64_t tok = t0 + c * C + i;
            const float *qt = q + (tok * H + h) * dk, *ktk = k + (tok * H + h) * dk;
            R dqs[DMO_DMAX];
            for (int64_t x = 0; x < dk; x++) dqs[x] = dqc[i * dk + x] * (R)p->scale;
            if (p->qk_l2norm) {
                R qs = 0, ks = 0;
                for (int64_t x = 0; x < dk; x++) {
                    qs += (R)qt[x] * (R)qt[x];
                    ks += (R)ktk[x] * (R)ktk[x];
                }
                R qi = (R)1 / SQRT(qs + (R)DMO_L2NORM_EPS), ki = (R)1 / SQRT(ks + (R)DMO_L2NORM_EPS);
                R sq = 0, sk = 0;
                for (int64_t x = 0; x < dk; x++) {
                    sq += (R)qt[x] * qi * dqs[x];
                    sk += (R)ktk[x] * ki * dkc[i * dk + x];
                }
                for (int64_t x = 0; x < dk; x++) {
                    dq_out[(tok * H + h) * dk + x] = (float)(qi * (dqs[x] - (R)qt[x] * qi * sq));
                    dk_out[(tok * H + h) * dk + x] =
                        (float)(ki * (dkc[i * dk + x] - (R)ktk[x] * ki * sk));
                }
            } else {
                for (int64_t x = 0; x < dk; x++) {
                    dq_out[(tok * H + h) * dk + x] = (float)dqs[x];
                    dk_out[(tok * H + h) * dk + x] = (float)dkc[i * dk + x];
                }
            }
            for (int64_t x = 0; x < dv; x++) dv_out[(tok * H + h) * dv + x] = (float)dvc[i * dv + x];
            dg_out[tok * H + h] = (float)dgc[i];
            dbeta_out[tok * H + h] = (float)d_beta[i];
        }
    }
    free(dqc); free(dkc); free(dvc); free(d_qg); free(dkt); free(dw); free(dkbg); free(dvb);
    free(dkbeta); free(vb); free(kbg); free(dattn); free(dT); free(m1); free(dA);
    free(ds); free(tmp); free(qg); free(attn); free(dvl);
    free(chs); free(states); free(vns); free(dos); free(ds_next); free(dvns);
}

int FN(dmo_gdr_chunk_bwd)(const dmo_gdr *p, const float *q, const float *k, const float *v,
                          const float *g, const float *beta, const float *h0,
                          const float *d_out, const float *d_final, float *dq, float *dk,
                          float *dv, float *dg, float *dbeta, float *dh0) {
    const int64_t S = p->cu ? p->nseq : p->b, H = p->h;
    if (p->dk > DMO_DMAX || p->dv > DMO_DMAX) return -1;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t r = 0; r < S * H; r++) {
        int64_t s = r / H, h = r % H, t0, len;
        FN(gdr_spans)(p, s, &t0, &len);
        if (len == 0) {
            /* an empty sequence passes its state, and the state's gradient, through */
            if (dh0)
                for (int64_t x = 0; x < p->dk * p->dv; x++)
                    dh0[r * p->dk * p->dv + x] = d_final ? d_final[r * p->dk * p->dv + x] : 0;
            continue;
        }
        FN(gdr_backward_one)(p, q, k, v, g, beta, h0, d_out, d_final, t0, len, h, r, dq, dk, dv,
                             dg, dbeta, dh0);
    }
    return 0;
}

#undef C

/* ------------------------------------------------------------------------------------------ */
/* Gated delta rule, recurrent step: crates/dash-ops/src/gated_delta/recurrent.rs:309-404      */
/* ------------------------------------------------------------------------------------------ */

/* `step` (:362-396) for every (sequence, head), packed sequences token by token (:318-358).
 * `state` [S, H, Dk, Dv] is advanced in place; out [T, H, Dv]. */
int FN(dmo_gdr_step)(const dmo_gdr *p, const float *q, const float *k, const float *v,
                     const float *g, const float *beta, float *state, float *out) {
    const int64_t S = p->cu ? p->nseq : p->b, H = p->h, dk = p->dk, dv = p->dv;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t r = 0; r < S * H; r++) {
        int64_t s = r / H, h = r % H;
        int64_t t0 = p->cu ? p->cu[s] : s, t1 = p->cu ? p->cu[s + 1] : s + 1;
        R *st = (R *)malloc(sizeof(R) * dk * dv);
        R *qn = (R *)malloc(sizeof(R) * dk), *kn = (R *)malloc(sizeof(R) * dk);
        R *kv = (R *)malloc(sizeof(R) * dv);
        for (int64_t x = 0; x < dk * dv; x++) st[x] = state[r * dk * dv + x];
        for (int64_t t = t0; t < t1; t++) {
            const float *qt = q + (t * H + h) * dk, *kt = k + (t * H + h) * dk;
            R qs = 0, ks = 0;
            for (int64_t x = 0; x < dk; x++) {
                qn[x] = qt[x];
                kn[x] = kt[x];
                qs += qn[x] * qn[x];
                ks += kn[x] * kn[x];
            }
            if (p->qk_l2norm) {
                R qi = (R)1 / SQRT(qs + (R)DMO_L2NORM_EPS), ki = (R)1 / SQRT(ks + (R)DMO_L2NORM_EPS);
                for (int64_t x = 0; x < dk; x++) {
                    qn[x] *= qi;
                    kn[x] *= ki;
                }
            }
            for (int64_t x = 0; x < dk; x++) qn[x] *= (R)p->scale;
            R decay = EXP((R)g[t * H + h]), bt = beta[t * H + h];
            for (int64_t x = 0; x < dk * dv; x++) st[x] *= decay;
            for (int64_t y = 0; y < dv; y++) {
                R acc = 0;
                for (int64_t x = 0; x < dk; x++) acc += st[x * dv + y] * kn[x];
                kv[y] = ((R)v[(t * H + h) * dv + y] - acc) * bt;
            }
            for (int64_t x = 0; x < dk; x++)
                for (int64_t y = 0; y < dv; y++) st[x * dv + y] += kn[x] * kv[y];
            for (int64_t y = 0; y < dv; y++) {
                R acc = 0;
                for (int64_t x = 0; x < dk; x++) acc += st[x * dv + y] * qn[x];
                out[(t * H + h) * dv + y] = (float)acc;
            }
        }
        for (int64_t x = 0; x < dk * dv; x++) state[r * dk * dv + x] = (float)st[x];
        free(st); free(qn); free(kn); free(kv);
    }
    return 0;
}

/* The step's gradients: reverse-mode differentiation of `step` (recurrent.rs:362-396) and of
 * `l2norm` (:400-404), as the reference's tracked step gets them from Burn's autodiff over the
 * same operations (:89-130), packed sequences token by token (:318-358). Each sequence's
 * per-token states are kept from a forward sweep, then the tokens are walked in reverse:
 *   S' = a P (a = exp g), kv = S'^T k, delta = beta (v - kv), S = S' + k delta^T, o = S^T qs;
 *   dS += qs dO^T;  dqs = S dO;  ddelta = dS^T k;  dkv = -beta ddelta;
 *   dk = dS delta + S' dkv;  dv = beta ddelta;  dbeta = ddelta . (v - kv);
 *   dS' = dS + k dkv^T;  dg = sum(dS' o S');  dP = a dS'.
 * d_out [T, H, Dv] and d_state [S, H, Dk, Dv] (NULL: zeros); d_state_in may be NULL. */
int FN(dmo_gdr_step_bwd)(const dmo_gdr *p, const float *q, const float *k, const float *v,
                         const float *g, const float *beta, const float *state,
                         const float *d_out, const float *d_state, float *dq, float *dk,
                         float *dv, float *dg, float *dbeta, float *d_state_in) {
    const int64_t S = p->cu ? p->nseq : p->b, H = p->h, dk_ = p->dk, dv_ = p->dv;
    const int64_t DD = dk_ * dv_;
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t r = 0; r < S * H; r++) {
        int64_t s = r / H, h = r % H;
        int64_t t0 = p->cu ? p->cu[s] : s, t1 = p->cu ? p->cu[s + 1] : s + 1;
        int64_t len = t1 - t0;
        /* pre[i]: the state before token t0 + i */
        R *pre = (R *)malloc(sizeof(R) * DD * (len > 0 ? len : 1));
        R *ds = (R *)malloc(sizeof(R) * DD), *sp = (R *)malloc(sizeof(R) * DD);
        R *qn = (R *)malloc(sizeof(R) * dk_), *kn = (R *)malloc(sizeof(R) * dk_);
        R *qi = (R *)malloc(sizeof(R) * (len > 0 ? len : 1)), *ki = (R *)malloc(sizeof(R) * (len > 0 ? len : 1));
        R *kv = (R *)malloc(sizeof(R) * dv_), *delta = (R *)malloc(sizeof(R) * dv_);
        R *ddelta = (R *)malloc(sizeof(R) * dv_), *dkv = (R *)malloc(sizeof(R) * dv_);
        R *dqs = (R *)malloc(sizeof(R) * dk_), *dkn = (R *)malloc(sizeof(R) * dk_);
        for (int64_t x = 0; x < DD; x++) {
            ds[x] = d_state ? (R)d_state[r * DD + x] : 0;
            if (len > 0) pre[x] = state[r * DD + x];
        }
        /* forward sweep: the normalised rows and the state before each token */
        for (int64_t i = 0; i < len; i++) {
            int64_t t = t0 + i;
            const float *qt = q + (t * H + h) * dk_, *kt = k + (t * H + h) * dk_;
            R qs = 0, ks = 0;
            for (int64_t x = 0; x < dk_; x++) {
                qs += (R)qt[x] * (R)qt[x];
                ks += (R)kt[x] * (R)kt[x];
            }
            qi[i] = p->qk_l2norm ? (R)1 / SQRT(qs + (R)DMO_L2NORM_EPS) : (R)1;
            ki[i] = p->qk_l2norm ? (R)1 / SQRT(ks + (R)DMO_L2NORM_EPS) : (R)1;
            if (i + 1 == len) break;
            R a = EXP((R)g[t * H + h]), bt = beta[t * H + h];
            const R *P = pre + i * DD;
            R *N = pre + (i + 1) * DD;
            for (int64_t x = 0; x < dk_; x++) kn[x] = (R)kt[x] * ki[i];
            for (int64_t y = 0; y < dv_; y++) {
                R acc = 0;
                for (int64_t x = 0; x < dk_; x++) acc += a * P[x * dv_ + y] * kn[x];
                delta[y] = ((R)v[(t * H + h) * dv_ + y] - acc) * bt;
            }
            for (int64_t x = 0; x < dk_; x++)
                for (int64_t y = 0; y < dv_; y++)
                    N[x * dv_ + y] = a * P[x * dv_ + y] + kn[x] * delta[y];
        }
        /* reverse sweep */
        for (int64_t i = len - 1; i >= 0; i--) {
            int64_t t = t0 + i;
            const float *qt = q + (t * H + h) * dk_, *kt = k + (t * H + h) * dk_;
            const float *vt = v + (t * H + h) * dv_;
            const float *dot = d_out ? d_out + (t * H + h) * dv_ : NULL;
            R a = EXP((R)g[t * H + h]), bt = beta[t * H + h];
            const R *P = pre + i * DD;
            for (int64_t x = 0; x < dk_; x++) {
                qn[x] = (R)qt[x] * qi[i] * (R)p->scale;
                kn[x] = (R)kt[x] * ki[i];
            }
            for (int64_t x = 0; x < DD; x++) sp[x] = a * P[x];
            for (int64_t y = 0; y < dv_; y++) {
                R acc = 0;
                for (int64_t x = 0; x < dk_; x++) acc += sp[x * dv_ + y] * kn[x];
                kv[y] = acc;
                delta[y] = ((R)vt[y] - acc) * bt;
            }
            /* o = S^T qs with S = S' + k delta^T */
            for (int64_t x = 0; x < dk_; x++) {
                R acc = 0;
                for (int64_t y = 0; y < dv_; y++) {
                    R o = dot ? (R)dot[y] : 0;
                    acc += (sp[x * dv_ + y] + kn[x] * delta[y]) * o;
                    ds[x * dv_ + y] += qn[x] * o;
                }
                dqs[x] = acc;
            }
            R db = 0;
            for (int64_t y = 0; y < dv_; y++) {
                R acc = 0;
                for (int64_t x = 0; x < dk_; x++) acc += ds[x * dv_ + y] * kn[x];
                ddelta[y] = acc;
                dkv[y] = -bt * acc;
                db += acc * ((R)vt[y] - kv[y]);
                dv[(t * H + h) * dv_ + y] = (float)(bt * acc);
            }
            R dgs = 0;
            for (int64_t x = 0; x < dk_; x++) {
                R acc = 0;
                for (int64_t y = 0; y < dv_; y++) {
                    acc += ds[x * dv_ + y] * delta[y] + sp[x * dv_ + y] * dkv[y];
                    R d1 = ds[x * dv_ + y] + kn[x] * dkv[y];
                    dgs += d1 * sp[x * dv_ + y];
                    ds[x * dv_ + y] = a * d1;
                }
                dkn[x] = acc;
            }
            dg[t * H + h] = (float)dgs;
            dbeta[t * H + h] = (float)db;
            /* through the scale and the l2 normalisation: d x = (d xn - xn (xn . d xn)) / n */
            R sq = 0, sk = 0;
            for (int64_t x = 0; x < dk_; x++) {
                dqs[x] *= (R)p->scale;
                sq += (R)qt[x] * qi[i] * dqs[x];
                sk += (R)kt[x] * ki[i] * dkn[x];
            }
            for (int64_t x = 0; x < dk_; x++) {
                if (p->qk_l2norm) {
                    dq[(t * H + h) * dk_ + x] = (float)(qi[i] * (dqs[x] - (R)qt[x] * qi[i] * sq));
                    dk[(t * H + h) * dk_ + x] = (float)(ki[i] * (dkn[x] - (R)kt[x] * ki[i] * sk));
                } else {
                    dq[(t * H + h) * dk_ + x] = (float)dqs[x];
                    dk[(t * H + h) * dk_ + x] = (float)dkn[x];
                }
            }
        }
        if (d_state_in)
            for (int64_t x = 0; x < DD; x++) d_state_in[r * DD + x] = (float)ds[x];
        free(pre); free(ds); free(sp); free(qn); free(kn); free(qi); free(ki); free(kv);
        free(delta); free(ddelta); free(dkv); free(dqs); free(dkn);
    }
    return 0;
}
