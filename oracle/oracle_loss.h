/* The fused linear cross-entropy, restated from crates/dash-ops/src/loss.rs and the gradient pass
 * of crates/dash-ops/src/logprob/reference.rs (TEST INFRASTRUCTURE ONLY; included twice by
 * dm_oracle.c, with R = float and R = double).
 *
 * Forward (loss.rs:411-525): the log-probability's pass over the vocabulary (oracle_logprob.h's
 * running m, s, r, a, zt, found) plus the sum of the unmasked logits, then per row
 *   lse = m + ln s;  logprob = zt - lse (-inf when the target is masked or out of range)
 *   loss = (1 - eps)(lse - zt) [+inf unseen; no term at eps = 1] + eps (lse - zsum / K)
 *          + lambda lse^2,  K the unmasked ids;  entropy = ln s - a / s;  q = r / s
 * with loss, logprob and entropy 0 on an ignored row. rows [8, n]: loss, logprob, entropy, lse,
 * q, s, counted, found (loss.rs:96-116 `row`).
 * Backward: the coefficients (loss.rs:597-668) from upstream [3, n] (the gradients of the loss,
 * logprob and entropy rows, 0 on an ignored row)
 *   A = gl (1 + 2 lambda lse) - gp - ge entropy
 *   T = gl (eps + 2 lambda lse) - q (gl (1 + 2 lambda lse) - gp) - (1 - q)(ge entropy + ge logprob)
 *       (0 unless found),  C = -gl eps / K
 * then the gradient pass (logprob/reference.rs:289-380): per chunk, the logits again and
 *   g = exp(z - lse)(A - E (z - lse)) + C,  g[t] = T + C,  g = 0 at a masked id
 * (E = ge when the entropy is asked for, else 0), grad_hidden += g weight_c,
 * grad_weight_c += g^T hidden. */

/* rows [8, n] (loss.rs:456-525 finish, over block_pass's sums). */
int FN(dmo_lce_fwd)(const dmo_lce *p, const float *hidden, const float *weight, float *rows) {
    const dmo_logprob *lp = &p->lp;
    const int64_t n = lp->n, v = lp->v, d = lp->d;
    if (n == 0) return 0;
    const int64_t nblocks = (n + lp->row_chunk - 1) / lp->row_chunk;
    const int64_t block = (n + nblocks - 1) / nblocks;
    const R K = (R)(v - lp->n_masked);
#pragma omp parallel
    {
        R *z = (R *)malloc(sizeof(R) * (size_t)v);
#pragma omp for schedule(dynamic, 1)
        for (int64_t i = 0; i < n; i++) {
            const int64_t r0 = (i / block) * block;
            const int64_t nrows = (r0 + block < n ? r0 + block : n) - r0;
            int64_t C = lp->vocab_chunk;
            if (C == 0) C = nrows < 2304 ? 4096 : 8192;
            const float *h = hidden + i * d;
            const int64_t t = lp->targets[i];
            R m = (R)(-3.4028234663852886e38), s = 0, r = 0, a = 0, zt = 0, found = 0, zsum = 0;
            for (int64_t c0 = 0; c0 < v; c0 += C) {
                const int64_t c1 = c0 + C < v ? c0 + C : v;
                R cmax = (R)(-3.4028234663852886e38);
                for (int64_t j = c0; j < c1; j++) {
                    R acc = 0;
                    for (int64_t e = 0; e < d; e++) acc += (R)h[e] * (R)weight[j * d + e];
                    z[j] = acc;
                    if (!FN(lp_is_masked)(lp, j) && acc > cmax) cmax = acc;
                }
                const R m_new = cmax > m ? cmax : m;
                const R shift = m - m_new, alpha = EXP(shift);
                R se = 0, sa = 0, sr = 0;
                for (int64_t j = c0; j < c1; j++) {
                    if (FN(lp_is_masked)(lp, j)) continue;
                    const R dz = z[j] - m_new, ej = EXP(dz);
                    se += ej;
                    sa += ej * dz;
                    zsum += z[j];
                    if (j == t) {
                        zt += z[j];
                        found += 1;
                        continue;
                    }
                    sr += ej;
                }
                a = alpha * (a + s * shift) + sa;
                s = s * alpha + se;
                r = r * alpha + sr;
                m = m_new;
            }
            const R ln_s = LOG(s), lse = m + ln_s;
            const int seen = found > (R)0.5, counted = t != p->ignore_index;
            const R eps = (R)p->eps, lam = (R)p->lambda;
            R loss = 0;
            if (eps < 1) loss = (1 - eps) * (seen ? lse - zt : (R)INFINITY);
            if (eps != 0) loss += eps * (lse - zsum / K);
            if (lam != 0) loss += lam * lse * lse;
            rows[0 * n + i] = counted ? (float)loss : 0.f;
            rows[1 * n + i] = counted ? (seen ? (float)(zt - lse) : -INFINITY) : 0.f;
            rows[2 * n + i] = counted ? (float)(ln_s - a / s) : 0.f;
            rows[3 * n + i] = (float)lse;
            rows[4 * n + i] = (float)(r / s);
            rows[5 * n + i] = (float)s;
            rows[6 * n + i] = counted ? 1.f : 0.f;
            rows[7 * n + i] = seen ? 1.f : 0.f;
        }
        free(z);
    }
    return 0;
}

/* grad_hidden [n, D] and grad_weight [V, D] (either may be NULL) from rows [8, n] and
 * upstream [3, n]. */
int FN(dmo_lce_bwd)(const dmo_lce *p, const float *hidden, const float *weight, const float *rows,
                    const float *upstream, float *grad_hidden, float *grad_weight) {
    const dmo_logprob *lp = &p->lp;
    const int64_t n = lp->n, v = lp->v, d = lp->d;
    if (grad_weight) memset(grad_weight, 0, sizeof(float) * (size_t)(v * d));
    if (n == 0) return 0;
    const R K = (R)(v - lp->n_masked), eps = (R)p->eps, lam = (R)p->lambda;
    /* the coefficients per row (loss.rs:597-668) */
    R *A = (R *)malloc(sizeof(R) * n), *T = (R *)malloc(sizeof(R) * n);
    R *E = (R *)malloc(sizeof(R) * n), *Cu = (R *)malloc(sizeof(R) * n);
    for (int64_t i = 0; i < n; i++) {
        const int counted = rows[6 * n + i] > 0.5f;
        const R gl = counted ? upstream[i] : 0, gp = counted ? upstream[n + i] : 0;
        const R ge = (p->entropy && counted) ? upstream[2 * n + i] : 0;
        const R lse = rows[3 * n + i], q = rows[4 * n + i];
        R soft = gl - gp;
        if (lam != 0) soft += gl * (lse * 2 * lam);
        R tgt = -q * soft;
        R glt = gl * eps;
        if (lam != 0) glt += gl * (lse * 2 * lam);
        tgt += glt;
        if (p->entropy) {
            const R ent = ge * (R)rows[2 * n + i];
            soft -= ent;
            const R pt = 1 - q;
            tgt -= pt * ent + ge * pt * (R)rows[n + i];
        }
        A[i] = soft;
        T[i] = rows[7 * n + i] > 0.5f ? tgt : 0;
        E[i] = ge;
        Cu[i] = -gl * eps / K;
    }
    /* the gradient pass: grad_hidden row by row; grad_weight summed over the rows in order */
    R *gw = grad_weight ? (R *)calloc((size_t)(v * d), sizeof(R)) : NULL;
    R *g = (R *)malloc(sizeof(R) * (size_t)v);
    R *gh = (R *)malloc(sizeof(R) * (size_t)d);
    for (int64_t i = 0; i < n; i++) {
        const float *h = hidden + i * d;
        const int64_t t = lp->targets[i];
        const R lse = rows[3 * n + i];
        for (int64_t j = 0; j < v; j++) {
            if (FN(lp_is_masked)(lp, j)) {
                g[j] = 0;
                continue;
            }
            if (j == t) {
                g[j] = T[i] + Cu[i];
                continue;
            }
            R acc = 0;
            for (int64_t e = 0; e < d; e++) acc += (R)h[e] * (R)weight[j * d + e];
            const R dz = acc - lse, pj = EXP(dz);
            g[j] = pj * (A[i] - E[i] * dz) + Cu[i];
        }
        if (grad_hidden) {
            for (int64_t e = 0; e < d; e++) gh[e] = 0;
            for (int64_t j = 0; j < v; j++)
                if (g[j] != 0)
                    for (int64_t e = 0; e < d; e++) gh[e] += g[j] * (R)weight[j * d + e];
            for (int64_t e = 0; e < d; e++) grad_hidden[i * d + e] = (float)gh[e];
        }
        if (gw) {
#pragma omp parallel for
            for (int64_t j = 0; j < v; j++)
                if (g[j] != 0)
                    for (int64_t e = 0; e < d; e++) gw[j * d + e] += g[j] * (R)h[e];
        }
    }
    if (gw) {
        for (int64_t x = 0; x < v * d; x++) grad_weight[x] = (float)gw[x];
        free(gw);
    }
    free(g);
    free(gh);
    free(A);
    free(T);
    free(E);
    free(Cu);
    return 0;
}
