/*
 * ORACLE - test infrastructure only.
 *
 * A plain-C restatement of the reference's exact-mode Lloyd pass, used as the checker for the HIP engine.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and only as
 * the checker or as the timed CPU baseline; the product path never calls it.
 *
 * What each function follows (citations are into the kakollu/mlx-kmeans reference):
 *   orc_assign     the rows loop that defines exact labels and best distances:
 *                  mlx_kmeans/core.py:263-274 (_ROWS_REG_SRC), identical to core.py:248-257 (_ROWS_SRC) and
 *                  to the argmin of the fused kernels core.py:1486-1495 and core.py:1577-1583.
 *                  s = 0; for j ascending: t = x_j - c_j; s += t*t; strict '<' over c ascending, so the lowest
 *                  index wins an exact tie; best = that s (float32).
 *                  Variant 0 (default, "A1"): product and add rounded separately, as the source reads (this
 *                  file is compiled with -ffp-contract=off). Variant 1: s = fma(t, t, s), the contracted form.
 *                  Which one Metal used cannot be read from the source; both are kept so a test can count
 *                  the labels that differ between them.
 *   orc_totals     per-cluster [count, sum of best, sum of x] (the totals layout of core.py:1629-1636 and
 *                  core.py:2018 `_gpu_pass`), accumulated in long double so it is exact to far below float32.
 *   orc_update     the host half of lloyd_step, core.py:2222-2242: counts = rint(tot[:,0]); inertia =
 *                  sum(tot[:,1]); empty clusters take the farthest rows (best descending, lower row index on
 *                  ties, paired with ascending empty ids; the order tests/accuracy.py:115-116 states); each
 *                  relocated row leaves its old cluster; centres = sums/counts rounded to float32; clusters
 *                  still empty take the largest cluster's centre (np.argmax: first maximum).
 *   orc_label_dist the direct-form distance of each row to a given label, the reference's kmeans_label_dist
 *                  (core.py:851-856), which the approximate path uses for best (core.py:1061-1088): the same
 *                  rows-loop arithmetic for one centre.
 *   orc_cpu_pass   the reference's native CPU backend, kmeans.mm:222-277 (cpu_block / assign_cpu): jobs of
 *                  CPU_BLOCK rows, each job a private float accumulator (count, best, x) on its own stack, the
 *                  job buffers reduced in double in job order. Threads replace GCD's dispatch_apply.
 *
 * Planted mutants (orc_assign `variant` 2..4) exist only so the tests can show that the pinning checks fail
 * on a plausible mistake: 2 = '<=' instead of '<' (highest index wins ties), 3 = last dimension dropped,
 * 4 = the row and centre swapped in the subtraction with the square replaced by t*|t| (a sign error).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_CPU_BLOCK 4096 /* rows per job, as kmeans.mm's CPU_BLOCK */

static float dist_variant(const float *x, const float *c, int d, int variant) {
    float s = 0.0f;
    if (variant == 1) {
        for (int j = 0; j < d; j++) { float t = x[j] - c[j]; s = fmaf(t, t, s); }
    } else if (variant == 3) {
        for (int j = 0; j < d - 1; j++) { float t = x[j] - c[j]; float p = t * t; s = s + p; }
    } else if (variant == 4) {
        for (int j = 0; j < d; j++) { float t = c[j] - x[j]; float p = t * fabsf(t); s = s + p; }
    } else {
        for (int j = 0; j < d; j++) { float t = x[j] - c[j]; float p = t * t; s = s + p; }
    }
    return s;
}

typedef struct {
    const float *X, *C;
    int64_t r0, r1;
    int d, k, variant;
    uint32_t *labels;
    float *best;
} assign_job;

static void *assign_worker(void *arg) {
    assign_job *a = (assign_job *)arg;
    for (int64_t i = a->r0; i < a->r1; i++) {
        const float *x = a->X + (size_t)i * a->d;
        float bst = INFINITY;
        uint32_t bl = 0;
        for (int c = 0; c < a->k; c++) {
            float s = dist_variant(x, a->C + (size_t)c * a->d, a->d, a->variant);
            int take = (a->variant == 2) ? (s <= bst) : (s < bst);
            if (take) { bst = s; bl = (uint32_t)c; }
        }
        if (a->labels) a->labels[i] = bl;
        if (a->best) a->best[i] = bst;
    }
    return NULL;
}

/* Exact nearest centre per row (see header). nthreads <= 0 means 1. */
void orc_assign(const float *X, int64_t n, int d, const float *C, int k, int variant, int nthreads,
                uint32_t *labels, float *best) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    pthread_t th[256];
    assign_job jobs[256];
    int64_t per = (n + nthreads - 1) / nthreads;
    int used = 0;
    for (int t = 0; t < nthreads; t++) {
        int64_t r0 = t * per, r1 = r0 + per < n ? r0 + per : n;
        if (r0 >= r1) break;
        jobs[t] = (assign_job){X, C, r0, r1, d, k, variant, labels, best};
        used++;
    }
    for (int t = 1; t < used; t++) pthread_create(&th[t], NULL, assign_worker, &jobs[t]);
    if (used > 0) assign_worker(&jobs[0]);
    for (int t = 1; t < used; t++) pthread_join(th[t], NULL);
}

/* out[i] = the rows-loop distance of row i to centre labels[i] (core.py:851-856). */
void orc_label_dist(const float *X, int64_t n, int d, const float *C, const uint32_t *labels, float *out) {
    for (int64_t i = 0; i < n; i++) out[i] = dist_variant(X + (size_t)i * d, C + (size_t)labels[i] * d, d, 0);
}

/* tot is (k, d+2) doubles: [count, sum best, sum x_0 .. sum x_{d-1}], summed in long double in row order. */
void orc_totals(const float *X, int64_t n, int d, const uint32_t *labels, const float *best, int k, double *tot) {
    int w = d + 2;
    long double *acc = (long double *)calloc((size_t)k * w, sizeof(long double));
    for (int64_t i = 0; i < n; i++) {
        long double *o = acc + (size_t)labels[i] * w;
        const float *x = X + (size_t)i * d;
        o[0] += 1.0L;
        o[1] += (long double)best[i];
        for (int j = 0; j < d; j++) o[2 + j] += (long double)x[j];
    }
    for (size_t e = 0; e < (size_t)k * w; e++) tot[e] = (double)acc[e];
    free(acc);
}

/* Farthest rows: the first m rows in the order (best descending, row ascending). Returns how many were
 * written (min(m, n)). Selection by repeated scan keeps this obviously right; m is small in every use. */
static int64_t farthest_rows(const float *best, int64_t n, int64_t m, int64_t *out) {
    int64_t got = 0;
    float prev_b = INFINITY;
    int64_t prev_r = -1;
    while (got < m && got < n) {
        int64_t pick = -1;
        float pb = -INFINITY;
        for (int64_t i = 0; i < n; i++) {
            float b = best[i];
            /* strictly after (prev_b, prev_r) in the order */
            int after = (b < prev_b) || (b == prev_b && i > prev_r);
            if (!after) continue;
            if (pick < 0 || b > pb) { pick = i; pb = b; }
        }
        if (pick < 0) break;
        out[got++] = pick;
        prev_b = pb;
        prev_r = pick;
    }
    return got;
}

/*
 * lloyd_step's host math (core.py:2222-2242) on totals `tot` (k, d+2) from a pass over X with centres C_in.
 * labels/best are that pass's. Writes C_out (k, d) float32, *inertia, *n_empty. tot is not modified.
 */
void orc_update(const double *tot, int k, int d, const float *X, int64_t n, const uint32_t *labels,
                const float *best, const float *C_in, float *C_out, double *inertia, int *n_empty) {
    (void)C_in;
    int w = d + 2;
    double *sums = (double *)malloc((size_t)k * d * sizeof(double));
    int64_t *counts = (int64_t *)malloc((size_t)k * sizeof(int64_t));
    double inert = 0.0;
    for (int c = 0; c < k; c++) {
        counts[c] = (int64_t)llrint(tot[(size_t)c * w]);
        inert += tot[(size_t)c * w + 1];
        for (int j = 0; j < d; j++) sums[(size_t)c * d + j] = tot[(size_t)c * w + 2 + j];
    }
    int m = 0;
    int *empty = (int *)malloc((size_t)k * sizeof(int));
    for (int c = 0; c < k; c++) if (counts[c] == 0) empty[m++] = c;   /* fixed before any relocation */
    if (m) {
        float bmax = 0.0f;
        for (int64_t i = 0; i < n; i++) if (best[i] > bmax) bmax = best[i];
        if (bmax > 0.0f) {
            int64_t *far = (int64_t *)malloc((size_t)m * sizeof(int64_t));
            int64_t got = farthest_rows(best, n, m, far);
            for (int64_t t = 0; t < got; t++) {
                int c = empty[t];
                int64_t f = far[t];
                uint32_t old = labels[f];
                const float *row = X + (size_t)f * d;
                for (int j = 0; j < d; j++) sums[(size_t)old * d + j] -= (double)row[j];
                counts[old] -= 1;
                for (int j = 0; j < d; j++) sums[(size_t)c * d + j] = (double)row[j];
                counts[c] = 1;
            }
            free(far);
        }
    }
    int big = 0;
    for (int c = 1; c < k; c++) if (counts[c] > counts[big]) big = c;
    for (int c = 0; c < k; c++) {
        if (counts[c] > 0)
            for (int j = 0; j < d; j++) C_out[(size_t)c * d + j] = (float)(sums[(size_t)c * d + j] / (double)counts[c]);
    }
    for (int c = 0; c < k; c++) {
        if (counts[c] <= 0)
            for (int j = 0; j < d; j++) C_out[(size_t)c * d + j] = C_out[(size_t)big * d + j];
    }
    *inertia = inert;
    *n_empty = m;
    free(empty);
    free(sums);
    free(counts);
}

/* ---- kmeans.mm's CPU backend (kmeans.mm:222-277), restated with pthreads ---- */
typedef struct {
    const float *X, *C;
    int d, k;
    int64_t n, njobs;
    int64_t *next;       /* shared job counter */
    pthread_mutex_t *mu;
    float *out;          /* njobs * k * (d+2) */
} cpu_pool;

static void cpu_block(const float *X, int64_t st, int64_t en, const float *C, int k, int d, float *out) {
    int W = d + 2;
    float *acc = (float *)calloc((size_t)k * W, sizeof(float));
    float *dist = (float *)malloc((size_t)k * sizeof(float));
    for (int64_t i = st; i < en; i++) {
        const float *x = X + (size_t)i * d;
        for (int c = 0; c < k; c++) {
            float s = 0;
            for (int j = 0; j < d; j++) { float t = x[j] - C[(size_t)c * d + j]; float p = t * t; s = s + p; }
            dist[c] = s;
        }
        int bl = 0;
        float bst = dist[0];
        for (int c = 1; c < k; c++) if (dist[c] < bst) { bst = dist[c]; bl = c; }
        float *o = acc + (size_t)bl * W;
        o[0] += 1;
        o[1] += bst;
        for (int j = 0; j < d; j++) o[2 + j] += x[j];
    }
    memcpy(out, acc, (size_t)k * W * sizeof(float));
    free(acc);
    free(dist);
}

static void *cpu_worker(void *arg) {
    cpu_pool *p = (cpu_pool *)arg;
    size_t kw = (size_t)p->k * (p->d + 2);
    for (;;) {
        pthread_mutex_lock(p->mu);
        int64_t j = (*p->next)++;
        pthread_mutex_unlock(p->mu);
        if (j >= p->njobs) break;
        int64_t st = j * ORC_CPU_BLOCK, en = st + ORC_CPU_BLOCK < p->n ? st + ORC_CPU_BLOCK : p->n;
        cpu_block(p->X, st, en, p->C, p->k, p->d, p->out + (size_t)j * kw);
    }
    return NULL;
}

/* One CPU pass: tot (k, d+2) doubles, job buffers reduced in double in job order. Returns 0 or -1. */
int orc_cpu_pass(const float *X, int64_t n, int d, const float *C, int k, int nthreads, double *tot) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    int64_t njobs = (n + ORC_CPU_BLOCK - 1) / ORC_CPU_BLOCK;
    size_t kw = (size_t)k * (d + 2);
    float *out = (float *)calloc((size_t)njobs * kw, sizeof(float));
    if (!out) return -1;
    int64_t next = 0;
    pthread_mutex_t mu = PTHREAD_MUTEX_INITIALIZER;
    cpu_pool p = {X, C, d, k, n, njobs, &next, &mu, out};
    pthread_t th[256];
    for (int t = 1; t < nthreads; t++) pthread_create(&th[t], NULL, cpu_worker, &p);
    cpu_worker(&p);
    for (int t = 1; t < nthreads; t++) pthread_join(th[t], NULL);
    for (size_t e = 0; e < kw; e++) tot[e] = 0.0;
    for (int64_t j = 0; j < njobs; j++)
        for (size_t e = 0; e < kw; e++) tot[e] += (double)out[(size_t)j * kw + e];
    free(out);
    return 0;
}
