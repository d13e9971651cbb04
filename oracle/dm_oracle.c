/* CPU oracle for the attention and gated-delta-rule hot path.
 *
 * TEST INFRASTRUCTURE ONLY: a plain-C restatement of dash-ops' reference implementations
 * (crates/dash-ops/src/attention/reference.rs, crates/dash-ops/src/gated_delta/chunk/reference.rs,
 * crates/dash-ops/src/gated_delta/recurrent.rs:309-404, crates/dash-ops/src/conv1d/reference.rs,
 * crates/dash-ops/src/logprob/reference.rs, crates/dash-ops/src/loss.rs),
 * compiled in f32 (the reference's own
 * precision, suffix _f32) and in f64 (suffix _f64). Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg load it, as the checker and as the timed CPU baseline; the product
 * library never links it.
 *
 * Parity of every function here is pinned by the reference's recorded fixtures
 * (tests/golden/, copied from crates/dash-ops/tests/fixtures/) and by brute-force checks in
 * tests/test_oracle.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define DMO_CHUNK 64
#define DMO_DMAX 256
#define DMO_L2NORM_EPS 1e-6f

typedef struct {
    int64_t b, tq, tk, hq, hkv, d;
    int32_t causal;
    float scale;
    /* window sides, -1 for unbounded (flash-attn's window_size; usize::MAX in the contract) */
    int64_t left, right;
    /* 0 none, 1 key padding [B, Tk] (nonzero = left out), 2 packed (cu_q, cu_k [nseq + 1]) */
    int32_t mask_kind;
    const uint8_t *padding;
    const int64_t *cu_q, *cu_k;
    int64_t nseq;
} dmo_attention;

typedef struct {
    int64_t b, t, h, dk, dv;
    const int64_t *cu; /* packed boundaries [nseq + 1] over a batch of one, or NULL */
    int64_t nseq;
    int32_t qk_l2norm;
    float scale;
} dmo_gdr;

/* One causal conv1d call (crates/dash-contract/src/conv1d.rs): x [B, T, C], weight [C, K],
 * bias [C], states [S, W, C]; packed sequences over a batch of one when cu is not NULL. */
typedef struct {
    int64_t b, t, c, k;
    const int64_t *cu; /* [nseq + 1] or NULL */
    int64_t nseq;
    int32_t has_bias, silu;
    int32_t has_h0;    /* initial states of w steps */
    int64_t w;
    int32_t has_final; /* final states of w_out steps */
    int64_t w_out;
} dmo_conv1d;

/* One chosen-token log-probability call (crates/dash-contract/src/logprob.rs): hidden [n, D],
 * weight [V, D], targets [n]; masked sorted and free of repeats; LogprobOptions. */
typedef struct {
    int64_t n, v, d;
    const int64_t *targets;
    const uint32_t *masked;
    int64_t n_masked;
    int64_t vocab_chunk, row_chunk;
} dmo_logprob;

/* One fused linear cross-entropy call (crates/dash-contract/src/loss.rs): the log-probability's
 * shapes, ids and chunks, and CrossEntropyOptions (reduction aside: the rows are per row). */
typedef struct {
    dmo_logprob lp;
    int64_t ignore_index;
    float eps, lambda;
    int32_t entropy;
} dmo_lce;

/* The sequence of `n` positions cut by `cu` [s + 1] that holds position `at`: the number of
 * ends at or before it, clamped into 0..s (reference.rs:118-159 `sequences`), and whether any
 * sequence holds it. */
static int64_t dmo_sequence_of(const int64_t *cu, int64_t s, int64_t at, int *inside) {
    int64_t idx = 0;
    for (int64_t x = 1; x <= s; x++)
        if (at >= cu[x]) idx++;
    *inside = at >= cu[0] && at < cu[s];
    if (idx > s - 1) idx = s - 1;
    return idx;
}

/* Whether key j is visible to query i of batch row b, element by element as the reference's
 * materialised mask says (reference.rs:91-112 `outside_window`, :163-222 `packed_hidden`,
 * :227-272 `hidden`). A window side binds only when it is below span = Tq + Tk + 1 (`bound`
 * :77-79); `reach` makes causality a right side of 0 (attention.rs:235-241). */
int dmo_attention_visible(const dmo_attention *a, int64_t b, int64_t i, int64_t j) {
    const int64_t span = a->tq + a->tk + 1;
    int64_t left = a->left, right = a->causal ? 0 : a->right;
    int has_left = left >= 0 && left < span, has_right = right >= 0 && right < span;
    int64_t pos, rel;
    if (a->mask_kind == 2) {
        int64_t s = a->nseq;
        if (s == 0 || a->tq == 0 || a->tk == 0) return 0;
        int in_q, in_k;
        int64_t sq = dmo_sequence_of(a->cu_q, s, i, &in_q);
        int64_t sk = dmo_sequence_of(a->cu_k, s, j, &in_k);
        if (sq != sk || !in_q || !in_k) return 0;
        int64_t q_start = a->cu_q[sq], q_len = a->cu_q[sq + 1] - q_start;
        int64_t k_start = a->cu_k[sq], k_len = a->cu_k[sq + 1] - k_start;
        pos = (i - q_start) + (k_len - q_len);
        rel = j - a->cu_k[sk];
    } else {
        pos = i + a->tk - a->tq;
        rel = j;
        if (a->mask_kind == 1 && a->padding[b * a->tk + j]) return 0;
    }
    if (has_right && rel > pos + right) return 0;
    if (has_left && rel < pos - left) return 0;
    return 1;
}

#define R float
#define FN(x) x##_f32
#define EXP expf
#define LOG logf
#define SQRT sqrtf
#include "oracle_body.h"
#include "oracle_conv1d.h"
#include "oracle_logprob.h"
#include "oracle_loss.h"
#undef R
#undef FN
#undef EXP
#undef LOG
#undef SQRT

#define R double
#define FN(x) x##_f64
#define EXP exp
#define LOG log
#define SQRT sqrt
#include "oracle_body.h"
#include "oracle_conv1d.h"
#include "oracle_logprob.h"
#include "oracle_loss.h"
#undef R
#undef FN
#undef EXP
#undef LOG
#undef SQRT

void dmo_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

int dmo_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
