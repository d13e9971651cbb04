/* The chosen-token log-probability and entropy, restated from
 * crates/dash-ops/src/logprob/reference.rs (TEST INFRASTRUCTURE ONLY; included twice by
 * dm_oracle.c, with R = float and R = double).
 *
 * For row i, logits z[i, j] = hidden[i] . weight[j] over the unmasked vocabulary
 * (crates/dash-contract/src/logprob.rs:4-15), walked in chunks of C tokens with the online
 * log-sum-exp of block_pass (reference.rs:226-287):
 *   m_new = max(m, max_j z),  shift = m - m_new,  alpha = exp(shift)   (m starts at f32::MIN)
 *   e_j   = exp(z_j - m_new)  (0 for a masked token)
 *   a     = alpha (a + s shift) + sum_j e_j (z_j - m_new)
 *   s     = alpha s + sum_j e_j;   r = alpha r + sum_{j != t} e_j
 *   o     = alpha o + sum_{j != t} e_j weight[j]                         (with the gradient)
 *   zt   += z_t, found += 1 when the target falls in the chunk unmasked
 * then (forward, reference.rs:96-120)
 *   logprob = zt - (m + ln s) where found, else -inf;  entropy = ln s - a / s
 *   grad    = (r found weight[t] - o) / s.
 * The rows are walked in blocks (RowBlocks, logprob.rs:105-111) whose size sets C
 * (VocabChunk, logprob.rs:90-101); each row's sums are independent of the others. Inputs are f32
 * values (already the dtype's values); the arithmetic is in R. */

static int FN(lp_is_masked)(const dmo_logprob *p, int64_t j) {
    /* masked is sorted and free of repeats (reference.rs:88 `sorted(masked)`) */
    int64_t lo = 0, hi = p->n_masked;
    while (lo < hi) {
        const int64_t mid = (lo + hi) / 2;
        if ((int64_t)p->masked[mid] < j) lo = mid + 1;
        else hi = mid;
    }
    return lo < p->n_masked && (int64_t)p->masked[lo] == j;
}

int FN(dmo_logprob)(const dmo_logprob *p, const float *hidden, const float *weight,
                    float *logprob, float *entropy, float *grad) {
    const int64_t n = p->n, v = p->v, d = p->d;
    if (n == 0) return 0;
    /* RowBlocks: as few blocks as row_chunk allows, of equal size but for the last */
    const int64_t nblocks = (n + p->row_chunk - 1) / p->row_chunk;
    const int64_t block = (n + (nblocks > 0 ? nblocks : 1) - 1) / (nblocks > 0 ? nblocks : 1);
#pragma omp parallel
    {
        R *z = (R *)malloc(sizeof(R) * (size_t)(v > 0 ? v : 1));
        R *o = (R *)malloc(sizeof(R) * (size_t)(d > 0 ? d : 1));
#pragma omp for schedule(dynamic, 1)
        for (int64_t i = 0; i < n; i++) {
            const int64_t r0 = (i / block) * block;
            const int64_t rows = (r0 + block < n ? r0 + block : n) - r0;
            int64_t C = p->vocab_chunk;
            if (C == 0) C = rows < 2304 ? 4096 : 8192;
            const float *h = hidden + i * d;
            const int64_t t = p->targets[i];
            R m = (R)(-3.4028234663852886e38), s = 0, r = 0, a = 0, zt = 0, found = 0;
            for (int64_t e = 0; e < d; e++) o[e] = 0;
            for (int64_t c0 = 0; c0 < v; c0 += C) {
                const int64_t c1 = c0 + C < v ? c0 + C : v;
                R cmax = (R)(-3.4028234663852886e38);
                for (int64_t j = c0; j < c1; j++) {
                    R acc = 0;
                    const float *w = weight + j * d;
                    for (int64_t e = 0; e < d; e++) acc += (R)h[e] * (R)w[e];
                    z[j] = acc;
                    if (!FN(lp_is_masked)(p, j) && acc > cmax) cmax = acc;
                }
                const R m_new = cmax > m ? cmax : m;
                const R shift = m - m_new, alpha = EXP(shift);
                R se = 0, sa = 0, sr = 0;
                if (grad)
                    for (int64_t e = 0; e < d; e++) o[e] *= alpha;
                for (int64_t j = c0; j < c1; j++) {
                    if (FN(lp_is_masked)(p, j)) continue;
                    const R dz = z[j] - m_new, ej = EXP(dz);
                    se += ej;
                    sa += ej * dz;
                    if (j == t) {
                        zt += z[j];
                        found += 1;
                        continue;
                    }
                    sr += ej;
                    if (grad) {
                        const float *w = weight + j * d;
                        for (int64_t e = 0; e < d; e++) o[e] += ej * (R)w[e];
                    }
                }
                a = alpha * (a + s * shift) + sa;
                s = s * alpha + se;
                r = r * alpha + sr;
                m = m_new;
            }
            const R ln_s = LOG(s);
            logprob[i] = found > (R)0.5 ? (float)(zt - (m + ln_s)) : -INFINITY;
            entropy[i] = (float)(ln_s - a / s);
            if (grad) {
                const R coef = r * found;
                const int in_range = t >= 0 && t < v;
                for (int64_t e = 0; e < d; e++) {
                    const R wt = in_range ? (R)weight[t * d + e] : 0;
                    grad[i * d + e] = (float)((wt * coef - o[e]) / s);
                }
            }
        }
        free(z);
        free(o);
    }
    return 0;
}
