/*
 * CPU oracle — TEST INFRASTRUCTURE ONLY (see kvc_oracle.h).
 *
 * Plain-C restatement of the reference's Linux CPU compaction path. Each
 * function names the reference lines it follows. The fp32 operation order
 * (sequential dot products, separate multiply and add, the same expf/sqrtf/
 * logf calls) is kept so results are bit-identical to the reference when
 * both are built with the same flags and libm; this is asserted by
 * tests/test_oracle.py against oracle/_ref and the golden fixtures.
 *
 * Parity status per function (all pinned bit-exactly against the compiled
 * reference on tests/golden fixtures unless noted):
 *   orc_kv_compact / _multi_round / _quantized, scoring, softmax-importance,
 *   top-t (libstdc++ heap-select restated), diversity greedy, GE LS solve,
 *   Lawson-Hanson NNLS, clamped-LS NNLS, refinement, quality stats, codec.
 *   orc_expf_replica: pinned against libm expf over every float in [-104, 0].
 */
#define _POSIX_C_SOURCE 199309L
#include "kvc_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static double now_ms(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e3 + ts.tv_nsec * 1e-6;
}

/* ------------------------------------------------------------------------ */
/* glibc expf restated. glibc >= 2.27 (x86-64, FMA ifunc) evaluates expf as  */
/* exp(x) = 2^(k/32) * 2^(r/32) with a 32-entry table of 2^(i/32) and a      */
/* cubic in double precision (ARM optimized-routines method, Szabolcs Nagy). */
/* The table is derived here from its definition; the GPU kernels use the   */
/* same restatement so softmax weights match the CPU bit for bit.           */
/* ------------------------------------------------------------------------ */
static uint64_t g_exp2_tab[32];

__attribute__((constructor)) static void exp2_tab_init(void) {
    /* tab[i] = bits(2^(i/32) rounded to nearest double) - (i << 47) */
    for (int i = 0; i < 32; i++) {
        /* 2^(i/32) to nearest double: exp2 in long double then round. */
        long double v = exp2l((long double)i / 32.0L);
        double d = (double)v;
        uint64_t b; memcpy(&b, &d, 8);
        g_exp2_tab[i] = b - ((uint64_t)i << 47);
    }
}

float orc_expf_replica(float x) {
    const double N = 32.0;
    const double inv_ln2_n = 0x1.71547652b82fep+0 * N;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / N / N / N;
    const double c1 = 0x1.ebfce50fac4f3p-3 / N / N;
    const double c2 = 0x1.62e42ff0c52d6p-1 / N;
    if (x < -0x1.9fe368p6f) return 0.0f;          /* underflows to +0 */
    if (x > 0x1.62e42ep6f) return HUGE_VALF;      /* overflow */
    double xd = (double)x;
    double z = inv_ln2_n * xd;
    double kd = z + shift;
    uint64_t ki; memcpy(&ki, &kd, 8);
    kd -= shift;
    double r = fma(inv_ln2_n, xd, -kd);
    uint64_t tb = g_exp2_tab[ki % 32] + (ki << 47);
    double s; memcpy(&s, &tb, 8);
    double p = fma(c0, r, c1);
    double r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(p, r2, y);
    return (float)(y * s);
}

/* ------------------------------------------------------------------------ */
/* dense helpers (reference include/kv-compact-math.h:44-263)               */
/* ------------------------------------------------------------------------ */

/* S[i][j] = (sum_l Q[i][l]*K[j][l]) * scale, sequential in l, then one
 * multiply (math.h:44-54 followed by api.cpp:626). Strided rows. */
void orc_scores(const float * Q, const float * K, float * S, int n_q, int T,
                int d, int stride_q, int stride_k, float scale) {
    for (int i = 0; i < n_q; i++) {
        const float * q = Q + (size_t)i * stride_q;
        for (int j = 0; j < T; j++) {
            const float * k = K + (size_t)j * stride_k;
            float acc = 0.0f;
            for (int l = 0; l < d; l++) acc += q[l] * k[l];
            S[(size_t)i * T + j] = acc;
        }
    }
    for (size_t i = 0; i < (size_t)n_q * T; i++) S[i] *= scale;
}

/* C[i][j] = sum_l A[i][l] * B[l][j], sequential in l (math.h:70-80), with
 * B's rows ldb floats apart: the reference's refit target Y_h = A_h V_h over
 * the head's slice of V (api.cpp:776-781 extracts the slice, then
 * mat_mul_AB; the same products in the same order). */
void orc_mat_mul_AB(const float * A, const float * B, float * C, int m, int k, int n, int ldb) {
    for (int i = 0; i < m; i++)
        for (int j = 0; j < n; j++) {
            float acc = 0.0f;
            for (int l = 0; l < k; l++) acc += A[(size_t)i * k + l] * B[(size_t)l * ldb + j];
            C[(size_t)i * n + j] = acc;
        }
}

/* softmax over rows, math.h:83-100 */
void orc_softmax_rows(float * x, int m, int n) {
    for (int i = 0; i < m; i++) {
        float * row = x + (size_t)i * n;
        float mx = row[0];
        for (int j = 1; j < n; j++) if (row[j] > mx) mx = row[j];
        float sum = 0.0f;
        for (int j = 0; j < n; j++) { row[j] = expf(row[j] - mx); sum += row[j]; }
        float inv = 1.0f / (sum + 1e-12f);
        for (int j = 0; j < n; j++) row[j] *= inv;
    }
}

/* fused row softmax + per-key importance, math.h:142-248 (both variants
 * share this arithmetic; exp_out/row_sums may be NULL). agg: 0 max, 1 rms,
 * 2 mean. */
void orc_softmax_importance(const float * S, float * attn, float * imp,
                            float * exp_out, float * row_sums, int m, int n, int agg) {
    memset(imp, 0, (size_t)n * sizeof(float));
    for (int i = 0; i < m; i++) {
        const float * row = S + (size_t)i * n;
        float * a = attn + (size_t)i * n;
        float mx = row[0];
        for (int j = 1; j < n; j++) if (row[j] > mx) mx = row[j];
        float sum = 0.0f;
        for (int j = 0; j < n; j++) {
            float e = expf(row[j] - mx);
            a[j] = e;
            if (exp_out) exp_out[(size_t)i * n + j] = e;
            sum += e;
        }
        if (row_sums) row_sums[i] = sum;
        float inv = 1.0f / (sum + 1e-12f);
        for (int j = 0; j < n; j++) {
            float sm = a[j] * inv;
            a[j] = sm;
            if (agg == 0) { if (sm > imp[j]) imp[j] = sm; }
            else if (agg == 1) imp[j] += sm * sm;
            else imp[j] += sm;
        }
    }
    if (agg == 1) {
        float inv_m = 1.0f / (float)m;
        for (int j = 0; j < n; j++) imp[j] = sqrtf(imp[j] * inv_m);
    } else if (agg == 2) {
        float inv_m = 1.0f / (float)m;
        for (int j = 0; j < n; j++) imp[j] *= inv_m;
    }
}

/* ------------------------------------------------------------------------ */
/* selection                                                                */
/* ------------------------------------------------------------------------ */

static int cmp_int(const void * a, const void * b) {
    int x = *(const int *)a, y = *(const int *)b;
    return (x > y) - (x < y);
}

/* std::partial_sort(first, first+k, last, greater-by-importance) keeps the
 * k-element set produced by libstdc++'s heap selection: build a heap over
 * the first k, then for each later element strictly more important than the
 * heap top, replace the top and sift. The set (not the order) is what the
 * reference keeps, since it sorts indices afterwards (api.cpp:727-742).
 * The heap routines below restate libstdc++'s __adjust_heap/__push_heap
 * (GCC 11) so that ties at the boundary resolve to the same members. */
static inline int heap_less(const float * imp, int a, int b) {
    /* the comparator passed to partial_sort: "a before b" */
    return imp[a] > imp[b];
}

static void heap_push(int * h, const float * imp, long hole, long top, int val) {
    long parent = (hole - 1) / 2;
    while (hole > top && heap_less(imp, h[parent], val)) {
        h[hole] = h[parent];
        hole = parent;
        parent = (hole - 1) / 2;
    }
    h[hole] = val;
}

static void heap_adjust(int * h, const float * imp, long hole, long len, int val) {
    const long top = hole;
    long child = hole;
    while (child < (len - 1) / 2) {
        child = 2 * (child + 1);
        if (heap_less(imp, h[child], h[child - 1])) child--;
        h[hole] = h[child];
        hole = child;
    }
    if ((len & 1) == 0 && child == (len - 2) / 2) {
        child = 2 * (child + 1);
        h[hole] = h[child - 1];
        hole = child - 1;
    }
    heap_push(h, imp, hole, top, val);
}

static void heap_select(int * a, long k, long n, const float * imp) {
    if (k >= 2) {
        long parent = (k - 2) / 2;
        for (;;) {
            int v = a[parent];
            heap_adjust(a, imp, parent, k, v);
            if (parent == 0) break;
            parent--;
        }
    }
    for (long i = k; i < n; i++) {
        if (heap_less(imp, a[i], a[0])) {
            int v = a[i];
            a[i] = a[0];
            heap_adjust(a, imp, 0, k, v);
        }
    }
}

/* top-t with forced prefix, api.cpp:716-744 */
int orc_select_topk(const float * imp, int T, int t, int n_prefix, int * out) {
    if (n_prefix > 0) {
        int pc = n_prefix < t ? n_prefix : t;
        int rem = t - pc;
        int nc = T - pc;
        int * cand = (int *)malloc((size_t)(nc > 0 ? nc : 1) * sizeof(int));
        for (int j = 0; j < nc; j++) cand[j] = pc + j;
        if (rem > 0) heap_select(cand, rem, nc, imp);
        for (int j = 0; j < pc; j++) out[j] = j;
        for (int j = 0; j < rem; j++) out[pc + j] = cand[j];
        free(cand);
    } else {
        int * idx = (int *)malloc((size_t)T * sizeof(int));
        for (int j = 0; j < T; j++) idx[j] = j;
        heap_select(idx, t, T, imp);
        memcpy(out, idx, (size_t)t * sizeof(int));
        free(idx);
    }
    qsort(out, (size_t)t, sizeof(int), cmp_int);
    return t;
}

/* cosine-diversity greedy, api.cpp:175-233. out_order (may be NULL) gets the
 * pick order before the final ascending sort. Returns the number kept. */
int orc_select_diverse(const float * imp, const float * K, int T, int t, int n_embd,
                       float strength, int n_prefix, int * out, int * out_order) {
    unsigned char * used = (unsigned char *)calloc((size_t)T, 1);
    float * pen = (float *)calloc((size_t)T, sizeof(float));
    int ns = 0;
    int pc = n_prefix < t ? n_prefix : t;
    for (int j = 0; j < pc; j++) { out[ns++] = j; used[j] = 1; }
    while (ns < t) {
        int best = -1;
        float best_score = -1e30f;
        for (int j = 0; j < T; j++) {
            if (used[j]) continue;
            float sc = imp[j] * (1.0f - strength * pen[j]);
            if (sc > best_score) { best_score = sc; best = j; }
        }
        if (best < 0) break;
        out[ns++] = best;
        used[best] = 1;
        const float * ks = K + (size_t)best * n_embd;
        float ns2 = 0.0f;
        for (int d = 0; d < n_embd; d++) ns2 += ks[d] * ks[d];
        ns2 = sqrtf(ns2) + 1e-8f;
        for (int j = 0; j < T; j++) {
            if (used[j]) continue;
            const float * kj = K + (size_t)j * n_embd;
            float dot = 0.0f, nj = 0.0f;
            for (int d = 0; d < n_embd; d++) { dot += ks[d] * kj[d]; nj += kj[d] * kj[d]; }
            float c = dot / (ns2 * sqrtf(nj) + 1e-8f);
            if (c > pen[j]) pen[j] = c;
        }
    }
    if (out_order) memcpy(out_order, out, (size_t)ns * sizeof(int));
    qsort(out, (size_t)ns, sizeof(int), cmp_int);
    free(used); free(pen);
    return ns;
}

/* ------------------------------------------------------------------------ */
/* solvers                                                                  */
/* ------------------------------------------------------------------------ */

/* Gaussian elimination with partial pivoting on [M | B] (n x (n+p)),
 * pivots below 1e-12 skipped; back substitution zeroes skipped rows.
 * Shared arithmetic of math.h:494-556, math.h:359-397, math.h:717-744.
 * zero_val is written for skipped pivots. */
static void ge_solve(float * aug, int n, int p, float * x, float zero_val) {
    const int w = n + p;
    for (int col = 0; col < n; col++) {
        int mr = col;
        float mv = fabsf(aug[(size_t)col * w + col]);
        for (int r = col + 1; r < n; r++) {
            float v = fabsf(aug[(size_t)r * w + col]);
            if (v > mv) { mv = v; mr = r; }
        }
        if (mr != col) {
            for (int j = 0; j < w; j++) {
                float tmp = aug[(size_t)col * w + j];
                aug[(size_t)col * w + j] = aug[(size_t)mr * w + j];
                aug[(size_t)mr * w + j] = tmp;
            }
        }
        float piv = aug[(size_t)col * w + col];
        if (fabsf(piv) < 1e-12f) continue;
        for (int r = col + 1; r < n; r++) {
            float f = aug[(size_t)r * w + col] / piv;
            for (int j = col; j < w; j++)
                aug[(size_t)r * w + j] -= f * aug[(size_t)col * w + j];
        }
    }
    for (int col = n - 1; col >= 0; col--) {
        float piv = aug[(size_t)col * w + col];
        if (fabsf(piv) < 1e-12f) {
            for (int j = 0; j < p; j++) x[(size_t)col * p + j] = zero_val;
            continue;
        }
        for (int j = 0; j < p; j++) {
            float v = aug[(size_t)col * w + n + j];
            for (int r = col + 1; r < n; r++) v -= aug[(size_t)col * w + r] * x[(size_t)r * p + j];
            x[(size_t)col * p + j] = v / piv;
        }
    }
}

/* ridge least squares via normal equations, math.h:463-557 */
void orc_ls_solve(const float * A, const float * b, float * x, int m, int n, int p, float ridge) {
    const int w = n + p;
    float * aug = (float *)malloc((size_t)n * w * sizeof(float));
    for (int i = 0; i < n; i++) {
        for (int j = 0; j < n; j++) {
            float s = 0.0f;
            for (int k = 0; k < m; k++) s += A[(size_t)k * n + i] * A[(size_t)k * n + j];
            aug[(size_t)i * w + j] = s;
        }
    }
    for (int i = 0; i < n; i++) aug[(size_t)i * w + i] += ridge;
    for (int i = 0; i < n; i++) {
        for (int l = 0; l < p; l++) {
            float s = 0.0f;
            for (int k = 0; k < m; k++) s += A[(size_t)k * n + i] * b[(size_t)k * p + l];
            aug[(size_t)i * w + n + l] = s;
        }
    }
    ge_solve(aug, n, p, x, 0.0f);
    free(aug);
}

static void gram_and_rhs(const float * A, const float * b, int m, int n, float * AtA, float * Atb) {
    for (int i = 0; i < n; i++)
        for (int j = 0; j < n; j++) {
            float s = 0.0f;
            for (int k = 0; k < m; k++) s += A[(size_t)k * n + i] * A[(size_t)k * n + j];
            AtA[(size_t)i * n + j] = s;
        }
    for (int i = 0; i < n; i++) {
        float s = 0.0f;
        for (int k = 0; k < m; k++) s += A[(size_t)k * n + i] * b[k];
        Atb[i] = s;
    }
}

/* the default NNLS method, math.h:683-806: clamped unconstrained LS (GE with
 * a 1e-10 ridge, skipped pivots give eps), then `iters` projected-gradient
 * steps of size 1 / L, L = u^T (A^T A) u after three power-iteration steps */
void orc_nnls_pgd(const float * A, const float * b, float * w, int m, int n, float eps, int iters) {
    float * AtA = (float *)malloc((size_t)n * n * sizeof(float));
    float * Atb = (float *)malloc((size_t)n * sizeof(float));
    gram_and_rhs(A, b, m, n, AtA, Atb);
    float * aug = (float *)malloc((size_t)n * (n + 1) * sizeof(float));
    for (int i = 0; i < n; i++) {
        for (int j = 0; j < n; j++) aug[(size_t)i * (n + 1) + j] = AtA[(size_t)i * n + j];
        aug[(size_t)i * (n + 1) + i] += 1e-10f;
        aug[(size_t)i * (n + 1) + n] = Atb[i];
    }
    ge_solve(aug, n, 1, w, eps);
    for (int i = 0; i < n; i++) if (w[i] < eps) w[i] = eps;
    free(aug);
    if (iters > 0) {
        float * u = (float *)malloc((size_t)n * sizeof(float));
        float * v = (float *)malloc((size_t)(m > 0 ? m : 1) * sizeof(float));
        float * grad = (float *)malloc((size_t)n * sizeof(float));
        for (int i = 0; i < n; i++) u[i] = 1.0f / sqrtf((float)n);
        for (int pw = 0; pw < 3; pw++) {
            for (int i = 0; i < m; i++) {
                float acc = 0.0f;
                for (int j = 0; j < n; j++) acc += A[(size_t)i * n + j] * u[j];
                v[i] = acc;
            }
            float vn = 0.0f;
            for (int i = 0; i < m; i++) vn += v[i] * v[i];
            vn = sqrtf(vn);
            if (vn < 1e-12f) break;
            for (int i = 0; i < m; i++) v[i] /= vn;
            for (int j = 0; j < n; j++) {
                float acc = 0.0f;
                for (int i = 0; i < m; i++) acc += A[(size_t)i * n + j] * v[i];
                u[j] = acc;
            }
            float un = 0.0f;
            for (int j = 0; j < n; j++) un += u[j] * u[j];
            un = sqrtf(un);
            if (un < 1e-12f) break;
            for (int j = 0; j < n; j++) u[j] /= un;
        }
        float L = 0.0f;
        for (int i = 0; i < n; i++) {
            float acc = 0.0f;
            for (int j = 0; j < n; j++) acc += AtA[(size_t)i * n + j] * u[j];
            L += u[i] * acc;
        }
        if (L < 1e-6f) L = 1e-6f;
        const float eta = 1.0f / L;
        for (int it = 0; it < iters; it++) {
            for (int i = 0; i < n; i++) {
                float acc = 0.0f;
                for (int j = 0; j < n; j++) acc += AtA[(size_t)i * n + j] * w[j];
                grad[i] = acc - Atb[i];
            }
            for (int i = 0; i < n; i++) {
                w[i] -= eta * grad[i];
                if (w[i] < eps) w[i] = eps;
            }
        }
        free(u); free(v); free(grad);
    }
    free(AtA); free(Atb);
}

void orc_nnls_clamped(const float * A, const float * b, float * w, int m, int n, float eps) {
    orc_nnls_pgd(A, b, w, m, n, eps, 0);
}

/* sensitivity of one head, math.h:579-594: largest over keys of the largest
 * weight over queries, over its mean */
float orc_head_sensitivity(const float * attn, int n_q, int T) {
    float sum_imp = 0.0f, max_imp = 0.0f;
    for (int j = 0; j < T; j++) {
        float max_w = 0.0f;
        for (int qi = 0; qi < n_q; qi++) {
            const float w = attn[(size_t)qi * T + j];
            if (w > max_w) max_w = w;
        }
        sum_imp += max_w;
        if (max_w > max_imp) max_imp = max_w;
    }
    const float mean_imp = sum_imp / (float)T;
    return max_imp / (mean_imp + 1e-12f);
}

static int cmp_sel_pair(const void * a, const void * b) {
    const int x = ((const int *)a)[0], y = ((const int *)b)[0];
    return (x > y) - (x < y);
}

/* OMP key selection, math.h:832-950: greedy picks by correlation with the
 * mass residual, NNLS refit (orc_nnls_pgd) every refit_interval iterations;
 * out sorted ascending with its weights; fewer than t picks are padded with
 * index 0 / weight 1e-12 */
void orc_omp_select(const float * E, const float * rs, int T, int n_q, int t, int * sel_out, float * w_out,
                    int k_choice, int refit_interval, int nnls_iters) {
    unsigned char * mask = (unsigned char *)calloc((size_t)T, 1);
    float * cur = (float *)calloc((size_t)(n_q > 0 ? n_q : 1), sizeof(float));
    float * res = (float *)malloc((size_t)(n_q > 0 ? n_q : 1) * sizeof(float));
    float * corr = (float *)malloc((size_t)T * sizeof(float));
    int * order = (int *)malloc((size_t)(t > 0 ? t : 1) * sizeof(int));
    float * prev_w = (float *)malloc((size_t)(t > 0 ? t : 1) * sizeof(float));
    float * M = (float *)malloc((size_t)(n_q > 0 ? n_q : 1) * (t > 0 ? t : 1) * sizeof(float));
    float * w = (float *)malloc((size_t)(t > 0 ? t : 1) * sizeof(float));
    int ns = 0, n_prev = 0, iteration = 0;
    while (ns < t) {
        for (int i = 0; i < n_q; i++) res[i] = rs[i] - cur[i];
        for (int j = 0; j < T; j++) {
            corr[j] = 0.0f;
            if (mask[j]) continue;
            float c = 0.0f;
            for (int i = 0; i < n_q; i++) c += E[(size_t)i * T + j] * res[i];
            corr[j] = c;
        }
        const int remaining = t - ns;
        int k_sel = k_choice < remaining ? k_choice : remaining;
        const int available = T - ns;
        if (k_sel > available) k_sel = available;
        if (k_sel <= 0) break;
        for (int k = 0; k < k_sel; k++) {
            int best = -1;
            float best_c = -1e30f;
            for (int j = 0; j < T; j++) {
                if (mask[j]) continue;
                if (corr[j] > best_c) { best_c = corr[j]; best = j; }
            }
            if (best < 0) break;
            order[ns++] = best;
            mask[best] = 1;
            corr[best] = -1e30f;
        }
        const int ct = ns;
        const int solve = (refit_interval <= 1) || (iteration % refit_interval == 0) || (ct == t);
        if (solve) {
            for (int i = 0; i < n_q; i++)
                for (int j = 0; j < ct; j++) M[(size_t)i * ct + j] = E[(size_t)i * T + order[j]];
            orc_nnls_pgd(M, rs, w, n_q, ct, 1e-12f, nnls_iters);
            for (int j = 0; j < ct; j++) prev_w[j] = w[j];
            n_prev = ct;
            for (int i = 0; i < n_q; i++) {
                float acc = 0.0f;
                for (int j = 0; j < ct; j++) acc += M[(size_t)i * ct + j] * w[j];
                cur[i] = acc;
            }
        } else {
            for (int j = n_prev; j < ct; j++) prev_w[j] = 1e-12f;
            n_prev = ct;
            for (int i = 0; i < n_q; i++) {
                float acc = 0.0f;
                for (int j = 0; j < ct; j++) acc += E[(size_t)i * T + order[j]] * prev_w[j];
                cur[i] = acc;
            }
        }
        iteration++;
    }
    /* sort by index, weights along (indices are distinct: a stable order is not needed) */
    int * pairs = (int *)malloc((size_t)(ns > 0 ? ns : 1) * 2 * sizeof(int));
    for (int j = 0; j < ns; j++) { pairs[2 * j] = order[j]; pairs[2 * j + 1] = j; }
    qsort(pairs, (size_t)ns, 2 * sizeof(int), cmp_sel_pair);
    for (int j = 0; j < ns; j++) {
        sel_out[j] = pairs[2 * j];
        if (w_out) w_out[j] = pairs[2 * j + 1] < n_prev ? prev_w[pairs[2 * j + 1]] : 1e-12f;
    }
    for (int j = ns; j < t; j++) {
        sel_out[j] = 0;
        if (w_out) w_out[j] = 1e-12f;
    }
    free(pairs); free(mask); free(cur); free(res); free(corr); free(order); free(prev_w); free(M); free(w);
}

/* Lawson-Hanson active set, math.h:283-452 */
void orc_nnls_lh(const float * A, const float * b, float * w, int m, int n, int max_iter) {
    float * AtA = (float *)malloc((size_t)n * n * sizeof(float));
    float * Atb = (float *)malloc((size_t)n * sizeof(float));
    gram_and_rhs(A, b, m, n, AtA, Atb);
    unsigned char * inP = (unsigned char *)calloc((size_t)n, 1);
    float * grad = (float *)malloc((size_t)n * sizeof(float));
    float * s = (float *)calloc((size_t)n, sizeof(float));
    int * pidx = (int *)malloc((size_t)n * sizeof(int));
    float * aug = (float *)malloc((size_t)n * (n + 1) * sizeof(float));
    float * sp = (float *)malloc((size_t)n * sizeof(float));
    for (int i = 0; i < n; i++) { w[i] = 0.0f; grad[i] = -Atb[i]; }
    for (int outer = 0; outer < max_iter; outer++) {
        int tix = -1;
        float md = 0.0f;
        for (int i = 0; i < n; i++)
            if (!inP[i] && (-grad[i]) > md) { md = -grad[i]; tix = i; }
        if (tix < 0 || md < 1e-10f) break;
        inP[tix] = 1;
        for (int inner = 0; inner < max_iter; inner++) {
            int pc = 0;
            for (int i = 0; i < n; i++) if (inP[i]) pidx[pc++] = i;
            for (int i = 0; i < pc; i++) {
                for (int j = 0; j < pc; j++)
                    aug[(size_t)i * (pc + 1) + j] = AtA[(size_t)pidx[i] * n + pidx[j]];
                aug[(size_t)i * (pc + 1) + i] += 1e-10f;
                aug[(size_t)i * (pc + 1) + pc] = Atb[pidx[i]];
            }
            ge_solve(aug, pc, 1, sp, 0.0f);
            for (int i = 0; i < n; i++) s[i] = 0.0f;
            for (int i = 0; i < pc; i++) s[pidx[i]] = sp[i];
            int feas = 1;
            for (int i = 0; i < pc; i++) if (sp[i] <= 0.0f) { feas = 0; break; }
            if (feas) { for (int i = 0; i < n; i++) w[i] = s[i]; break; }
            float alpha = 1.0f;
            for (int i = 0; i < pc; i++) {
                int ix = pidx[i];
                if (s[ix] <= 0.0f) {
                    float a = w[ix] / (w[ix] - s[ix] + 1e-30f);
                    if (a < alpha) alpha = a;
                }
            }
            for (int i = 0; i < n; i++) w[i] += alpha * (s[i] - w[i]);
            for (int i = 0; i < pc; i++) {
                int ix = pidx[i];
                if (fabsf(w[ix]) < 1e-12f) { w[ix] = 0.0f; inP[ix] = 0; }
            }
        }
        for (int i = 0; i < n; i++) {
            float acc = 0.0f;
            for (int j = 0; j < n; j++) acc += AtA[(size_t)i * n + j] * w[j];
            grad[i] = acc - Atb[i];
        }
    }
    for (int i = 0; i < n; i++) if (w[i] < 1e-12f) w[i] = 1e-12f;
    free(AtA); free(Atb); free(inP); free(grad); free(s); free(pidx); free(aug); free(sp);
}

/* ------------------------------------------------------------------------ */
/* quality statistics, api.cpp:239-325                                       */
/* ------------------------------------------------------------------------ */
void orc_quality_stats(const float * K, const float * V, const float * Q, int T, int n_q,
                       int H, int d_k, int d_v, const kv_compact_result * r,
                       kv_compact_stats * st) {
    float inv = 1.0f / sqrtf((float)d_k);
    int t = r->t;
    int ek = H * d_k, ev = H * d_v;
    float sum_cos = 0.0f, sum_mse = 0.0f;
    int agree = 0, total = 0;
    int mh = H < 4 ? H : 4;
    int mq = n_q < 32 ? n_q : 32;
    float * os = (float *)malloc((size_t)T * sizeof(float));
    float * cs = (float *)malloc((size_t)(t > 0 ? t : 1) * sizeof(float));
    float * oo = (float *)malloc((size_t)d_v * sizeof(float));
    float * co = (float *)malloc((size_t)d_v * sizeof(float));
    for (int h = 0; h < mh; h++) {
        for (int qi = 0; qi < mq; qi++) {
            const float * q = Q + (size_t)qi * ek + (size_t)h * d_k;
            for (int j = 0; j < T; j++) {
                const float * k = K + (size_t)j * ek + (size_t)h * d_k;
                float dot = 0.0f;
                for (int d = 0; d < d_k; d++) dot += q[d] * k[d];
                os[j] = dot * inv;
            }
            orc_softmax_rows(os, 1, T);
            for (int d = 0; d < d_v; d++) oo[d] = 0.0f;
            for (int j = 0; j < T; j++) {
                const float * v = V + (size_t)j * ev + (size_t)h * d_v;
                for (int d = 0; d < d_v; d++) oo[d] += os[j] * v[d];
            }
            for (int j = 0; j < t; j++) {
                const float * k = K + (size_t)r->selected_indices[j] * ek + (size_t)h * d_k;
                float dot = 0.0f;
                for (int d = 0; d < d_k; d++) dot += q[d] * k[d];
                cs[j] = dot * inv + r->beta[h][j];
            }
            orc_softmax_rows(cs, 1, t);
            for (int d = 0; d < d_v; d++) co[d] = 0.0f;
            for (int j = 0; j < t; j++)
                for (int d = 0; d < d_v; d++) co[d] += cs[j] * r->C_v[h][(size_t)j * d_v + d];
            float dp = 0.0f, no = 0.0f, nc = 0.0f;
            for (int d = 0; d < d_v; d++) { dp += oo[d] * co[d]; no += oo[d] * oo[d]; nc += co[d] * co[d]; }
            sum_cos += dp / (sqrtf(no * nc) + 1e-8f);
            float mse = 0.0f;
            for (int d = 0; d < d_v; d++) { float df = oo[d] - co[d]; mse += df * df; }
            sum_mse += mse / d_v;
            int ao = 0, ac = 0;
            for (int d = 1; d < d_v; d++) {
                if (oo[d] > oo[ao]) ao = d;
                if (co[d] > co[ac]) ac = d;
            }
            if (ao == ac) agree++;
            total++;
        }
    }
    st->avg_cosine_sim = sum_cos / total;
    st->avg_mse = sum_mse / total;
    st->avg_agreement = (float)agree / total;
    free(os); free(cs); free(oo); free(co);
}

/* ------------------------------------------------------------------------ */
/* orchestration, api.cpp:333-978                                            */
/* ------------------------------------------------------------------------ */

kv_compact_params orc_params_default(void) {
    kv_compact_params p;
    memset(&p, 0, sizeof(p));
    p.target_ratio = 0.5f;
    p.ridge = 1e-6f;
    p.nnls_max_iter = 200;
    p.diversity_strength = 0.5f;
    p.skip_beta = 1;
    p.score_method = 1;
    p.omp_k_choice = 1;
    p.omp_refit_interval = 1;
    p.nnls_method = 1;
    return p;
}

/* api.cpp:132-152 with the sizing of api.cpp:382-390 */
static int cheap_qref_count(int T) {
    int n = T / 2;
    if (n > 64) n = 64;
    if (n < 4) n = 4;
    if (n > T) n = T;
    return n;
}

static float * make_cheap_qref(const float * K, int T, int ek, int n) {
    float * Q = (float *)malloc((size_t)n * ek * sizeof(float));
    for (int qi = 0; qi < n; qi++) {
        float f = (float)(qi + 1) / (float)(n + 1);
        f = f * f;
        int pos = (int)(f * (T - 1));
        if (pos >= T) pos = T - 1;
        if (pos < 0) pos = 0;
        memcpy(Q + (size_t)qi * ek, K + (size_t)pos * ek, (size_t)ek * sizeof(float));
    }
    return Q;
}

int orc_target_count(int T, const kv_compact_params * p) {
    int t;
    if (p->target_count > 0) {
        t = p->target_count < T ? p->target_count : T;
    } else {
        t = (int)(T * p->target_ratio);
        if (t < 1) t = 1;
        if (t > T) t = T;
    }
    if (p->n_shared_prefix > t) t = p->n_shared_prefix < T ? p->n_shared_prefix : T;
    return t;
}

int orc_chunk_plan(int T, const kv_compact_params * p, int * chunk_out) {
    int cs = p->chunk_size;
    if (cs == 0) {
        float r = (p->target_count > 0) ? (float)p->target_count / (float)T : p->target_ratio;
        if (r <= 0.0f) r = 0.5f;
        if (r > 1.0f) r = 1.0f;
        int est = (int)(T * r);
        if (est > 256) {
            cs = (int)(256.0f / r);
            if (cs < 64) cs = 64;
            if (cs >= T) cs = T;
        } else {
            cs = T;
        }
    } else if (cs < 0) {
        cs = T;
    }
    *chunk_out = cs;
    return (T + cs - 1) / cs;
}

static void free_partial(float ** a, int n) {
    if (!a) return;
    for (int i = 0; i < n; i++) free(a[i]);
    free(a);
}

/* beta for one head, api.cpp:791-831 */
static void solve_beta(const float * expS, const float * row_sums, const int * sel,
                       int n_q, int T, int t, const kv_compact_params * p, float * beta) {
    if (p->skip_beta) { for (int j = 0; j < t; j++) beta[j] = 0.0f; return; }
    float * M = (float *)malloc((size_t)n_q * t * sizeof(float));
    float * w = (float *)malloc((size_t)t * sizeof(float));
    for (int qi = 0; qi < n_q; qi++)
        for (int j = 0; j < t; j++) M[(size_t)qi * t + j] = expS[(size_t)qi * T + sel[j]];
    if (p->nnls_method == 0) orc_nnls_lh(M, row_sums, w, n_q, t, p->nnls_max_iter);
    else orc_nnls_pgd(M, row_sums, w, n_q, t, 1e-12f, p->nnls_pgd_iters);
    for (int j = 0; j < t; j++) {
        float v = (1e-12f < w[j]) ? w[j] : 1e-12f;   /* std::max(1e-12f, w) */
        beta[j] = logf(v);
    }
    free(M); free(w);
}

/* X = softmax(S[:, sel] + beta), then ridge LS, api.cpp:833-848 */
static void refit_values(const float * S, const int * sel, const float * beta, const float * Y,
                         int n_q, int T, int t, int d_v, float ridge, float * Cv) {
    float * X = (float *)malloc((size_t)n_q * t * sizeof(float));
    for (int qi = 0; qi < n_q; qi++)
        for (int j = 0; j < t; j++) X[(size_t)qi * t + j] = S[(size_t)qi * T + sel[j]] + beta[j];
    orc_softmax_rows(X, n_q, t);
    orc_ls_solve(X, Y, Cv, n_q, t, d_v, ridge);
    free(X);
}

/* one unchunked call body, api.cpp:562-977 */
static int compact_body(const float * K, const float * V, const float * Q, int T, int n_q,
                        int H, int d_k, int d_v, const kv_compact_params * p, int t,
                        kv_compact_result * res) {
    double t0 = now_ms();
    const int ek = H * d_k, ev = H * d_v;
    const float inv_sqrt = 1.0f / sqrtf((float)d_k);
    const int need_exp = !p->skip_beta || p->use_omp;   /* OMP reads the exp scores (api.cpp:634-643) */
    float * S = (float *)malloc((size_t)H * n_q * T * sizeof(float));
    float * A = (float *)malloc((size_t)H * n_q * T * sizeof(float));
    float * E = need_exp ? (float *)malloc((size_t)H * n_q * T * sizeof(float)) : NULL;
    float * RS = need_exp ? (float *)malloc((size_t)H * n_q * sizeof(float)) : NULL;
    float * gimp = (float *)calloc((size_t)T, sizeof(float));
    float * himp = (float *)malloc((size_t)T * H * sizeof(float));
    float * sens = (float *)malloc((size_t)H * sizeof(float));
    for (int h = 0; h < H; h++) {
        float * Sh = S + (size_t)h * n_q * T;
        float * ih = himp + (size_t)h * T;
        orc_scores(Q + (size_t)h * d_k, K + (size_t)h * d_k, Sh, n_q, T, d_k, ek, ek, inv_sqrt);
        orc_softmax_importance(Sh, A + (size_t)h * n_q * T, ih,
                               E ? E + (size_t)h * n_q * T : NULL,
                               RS ? RS + (size_t)h * n_q : NULL, n_q, T, p->score_method);
        if (p->use_sensitivity) sens[h] = orc_head_sensitivity(A + (size_t)h * n_q * T, n_q, T);
        else for (int j = 0; j < T; j++) if (ih[j] > gimp[j]) gimp[j] = ih[j];
    }
    /* sensitivity weighting, math.h:605-618: out[j] += s_h * imp_h[j], heads in order */
    if (p->use_sensitivity)
        for (int h = 0; h < H; h++)
            for (int j = 0; j < T; j++) gimp[j] += sens[h] * himp[(size_t)h * T + j];
    if (p->reasoning && p->reasoning->classifier) {
        const kv_compact_reasoning * rk = p->reasoning;
        for (int j = 0; j < T; j++) {
            int ty = rk->classifier(j + rk->token_offset, rk->classifier_data);
            float wgt = 1.0f;
            if (ty == KV_TOKEN_THINKING) wgt = rk->thinking_weight;
            else if (ty == KV_TOKEN_TRANSITION) wgt = rk->transition_weight;
            gimp[j] *= wgt;
        }
    }
    int * sel = (int *)malloc((size_t)t * sizeof(int));
    if (p->use_omp) {
        /* OMP on the exp scores and row sums summed over heads, api.cpp:690-711 */
        float * ce = (float *)calloc((size_t)n_q * T, sizeof(float));
        float * cs = (float *)calloc((size_t)(n_q > 0 ? n_q : 1), sizeof(float));
        for (int h = 0; h < H; h++) {
            for (size_t i = 0; i < (size_t)n_q * T; i++) ce[i] += E[(size_t)h * n_q * T + i];
            for (int i = 0; i < n_q; i++) cs[i] += RS[(size_t)h * n_q + i];
        }
        orc_omp_select(ce, cs, T, n_q, t, sel, NULL, p->omp_k_choice, p->omp_refit_interval, p->nnls_pgd_iters);
        free(ce); free(cs);
    } else if (p->use_diversity) {
        t = orc_select_diverse(gimp, K, T, t, ek, p->diversity_strength, p->n_shared_prefix, sel, NULL);
    } else {
        orc_select_topk(gimp, T, t, p->n_shared_prefix, sel);
    }
    double scoring_ms = now_ms() - t0;
    double t1 = now_ms();

    /* Y_h = A_h V_h, math.h:70-80 */
    float * Y = (float *)malloc((size_t)H * n_q * d_v * sizeof(float));
    for (int h = 0; h < H; h++) {
        const float * Ah = A + (size_t)h * n_q * T;
        for (int i = 0; i < n_q; i++)
            for (int c = 0; c < d_v; c++) {
                float s = 0.0f;
                for (int l = 0; l < T; l++) s += Ah[(size_t)i * T + l] * V[(size_t)l * ev + (size_t)h * d_v + c];
                Y[((size_t)h * n_q + i) * d_v + c] = s;
            }
    }
    float * beta = (float *)malloc((size_t)H * t * sizeof(float));
    float * Cv = (float *)malloc((size_t)H * t * d_v * sizeof(float));
    for (int h = 0; h < H; h++) {
        solve_beta(E ? E + (size_t)h * n_q * T : NULL, RS ? RS + (size_t)h * n_q : NULL, sel,
                   n_q, T, t, p, beta + (size_t)h * t);
        refit_values(S + (size_t)h * n_q * T, sel, beta + (size_t)h * t,
                     Y + (size_t)h * n_q * d_v, n_q, T, t, d_v, p->ridge, Cv + (size_t)h * t * d_v);
    }

    /* refinement rounds, api.cpp:851-946 */
    if (p->refine_rounds > 0 && t < T) {
        unsigned char * is_sel = (unsigned char *)calloc((size_t)T, 1);
        for (int j = 0; j < t; j++) is_sel[sel[j]] = 1;
        float * kv = (float *)malloc((size_t)t * sizeof(float));
        float * row = (float *)malloc((size_t)t * sizeof(float));
        float * err = (float *)malloc((size_t)t * sizeof(float));
        for (int rr = 0; rr < p->refine_rounds; rr++) {
            for (int j = 0; j < t; j++) kv[j] = 0.0f;
            for (int h = 0; h < H; h++) {
                const float * Sh = S + (size_t)h * n_q * T;
                const float * bh = beta + (size_t)h * t;
                for (int j = 0; j < t; j++) err[j] = 0.0f;
                for (int qi = 0; qi < n_q; qi++) {
                    for (int j = 0; j < t; j++) row[j] = Sh[(size_t)qi * T + sel[j]] + bh[j];
                    orc_softmax_rows(row, 1, t);
                    for (int j = 0; j < t; j++) err[j] += row[j] * row[j];
                }
                for (int j = 0; j < t; j++) kv[j] += err[j] / n_q;
            }
            int worst = 0;
            for (int j = 1; j < t; j++) if (kv[j] < kv[worst]) worst = j;
            int bu = -1;
            float bi = -1.0f;
            for (int j = 0; j < T; j++)
                if (!is_sel[j] && gimp[j] > bi) { bi = gimp[j]; bu = j; }
            if (bu < 0) break;
            if (bi <= gimp[sel[worst]] * 0.5f) break;
            is_sel[sel[worst]] = 0;
            is_sel[bu] = 1;
            sel[worst] = bu;
            qsort(sel, (size_t)t, sizeof(int), cmp_int);
            for (int h = 0; h < H; h++) {
                solve_beta(E ? E + (size_t)h * n_q * T : NULL, RS ? RS + (size_t)h * n_q : NULL,
                           sel, n_q, T, t, p, beta + (size_t)h * t);
                refit_values(S + (size_t)h * n_q * T, sel, beta + (size_t)h * t,
                             Y + (size_t)h * n_q * d_v, n_q, T, t, d_v, p->ridge,
                             Cv + (size_t)h * t * d_v);
            }
        }
        free(is_sel); free(kv); free(row); free(err);
    }
    double nnls_ms = now_ms() - t1;

    res->t = t;
    res->n_head_kv = H;
    res->selected_indices = sel;
    res->beta = (float **)malloc((size_t)H * sizeof(float *));
    res->C_v = (float **)malloc((size_t)H * sizeof(float *));
    for (int h = 0; h < H; h++) {
        res->beta[h] = (float *)malloc((size_t)t * sizeof(float));
        memcpy(res->beta[h], beta + (size_t)h * t, (size_t)t * sizeof(float));
        res->C_v[h] = (float *)malloc((size_t)t * d_v * sizeof(float));
        memcpy(res->C_v[h], Cv + (size_t)h * t * d_v, (size_t)t * d_v * sizeof(float));
    }
    orc_quality_stats(K, V, Q, T, n_q, H, d_k, d_v, res, &res->stats);
    res->stats.elapsed_ms = now_ms() - t0;
    res->stats.scoring_ms = scoring_ms;
    res->stats.nnls_ms = nnls_ms;
    free(S); free(A); free(E); free(RS); free(gimp); free(himp); free(sens); free(Y); free(beta); free(Cv);
    return 0;
}

static int compact_impl(const float * K, const float * V, const float * Q, int T, int n_q,
                        int H, int d_k, int d_v, const kv_compact_params * params,
                        kv_compact_result * res);

/* chunked path, api.cpp:439-560 */
static int compact_chunked(const float * K, const float * V, const float * Qu, int T, int nqu,
                           int H, int d_k, int d_v, const kv_compact_params * p, int cs,
                           kv_compact_result * res) {
    double t0 = now_ms();
    const int ek = H * d_k, ev = H * d_v;
    int nc = (T + cs - 1) / cs;
    kv_compact_result * cr = (kv_compact_result *)calloc((size_t)nc, sizeof(kv_compact_result));
    int * rc = (int *)calloc((size_t)nc, sizeof(int));
    int nth = p->n_threads;
#ifdef _OPENMP
    if (nth <= 0) nth = omp_get_max_threads();
    if (nth > nc) nth = nc;
#else
    nth = 1;
#endif
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic) num_threads(nth) if (nth > 1)
#endif
    for (int c = 0; c < nc; c++) {
        int start = c * cs;
        int end = start + cs < T ? start + cs : T;
        int cT = end - start;
        kv_compact_params cp = *p;
        cp.chunk_size = -1;
        cp.n_threads = 1;
        if (c > 0) cp.n_shared_prefix = 0;
        if (cp.n_shared_prefix > cT) cp.n_shared_prefix = cT;
        kv_compact_reasoning crk;
        if (cp.reasoning) {
            crk = *cp.reasoning;
            crk.token_offset += start;
            cp.reasoning = &crk;
        }
        rc[c] = compact_impl(K + (size_t)start * ek, V + (size_t)start * ev, Qu, cT, nqu,
                             H, d_k, d_v, &cp, &cr[c]);
    }
    for (int c = 0; c < nc; c++) {
        if (rc[c] != 0) {
            int e = rc[c];
            for (int i = 0; i < nc; i++) orc_result_free(&cr[i]);
            free(cr); free(rc);
            return e;
        }
    }
    int tot = 0;
    for (int c = 0; c < nc; c++) tot += cr[c].t;
    res->t = tot;
    res->n_head_kv = H;
    res->selected_indices = (int *)malloc((size_t)tot * sizeof(int));
    res->beta = (float **)malloc((size_t)H * sizeof(float *));
    res->C_v = (float **)malloc((size_t)H * sizeof(float *));
    for (int h = 0; h < H; h++) {
        res->beta[h] = (float *)malloc((size_t)tot * sizeof(float));
        res->C_v[h] = (float *)malloc((size_t)tot * d_v * sizeof(float));
    }
    int off = 0;
    for (int c = 0; c < nc; c++) {
        for (int j = 0; j < cr[c].t; j++) res->selected_indices[off + j] = cr[c].selected_indices[j] + c * cs;
        for (int h = 0; h < H; h++) {
            memcpy(res->beta[h] + off, cr[c].beta[h], (size_t)cr[c].t * sizeof(float));
            memcpy(res->C_v[h] + (size_t)off * d_v, cr[c].C_v[h], (size_t)cr[c].t * d_v * sizeof(float));
        }
        off += cr[c].t;
    }
    orc_quality_stats(K, V, Qu, T, nqu, H, d_k, d_v, res, &res->stats);
    res->stats.elapsed_ms = now_ms() - t0;
    double ss = 0.0, sn = 0.0;
    for (int c = 0; c < nc; c++) { ss += cr[c].stats.scoring_ms; sn += cr[c].stats.nnls_ms; }
    res->stats.scoring_ms = ss;
    res->stats.nnls_ms = sn;
    for (int c = 0; c < nc; c++) orc_result_free(&cr[c]);
    free(cr); free(rc);
    return 0;
}

static int compact_impl(const float * K, const float * V, const float * Q, int T, int n_q,
                        int H, int d_k, int d_v, const kv_compact_params * params,
                        kv_compact_result * res) {
    if (!K || !V || !res) return -1;
    if (T <= 0 || H <= 0 || d_k <= 0 || d_v <= 0) return -2;
    kv_compact_params p = params ? *params : orc_params_default();
    const int ek = H * d_k;
    float * cheap = NULL;
    const float * Qu = Q;
    int nqu = n_q;
    if (p.use_cheap_qref || !Q) {
        nqu = cheap_qref_count(T);
        cheap = make_cheap_qref(K, T, ek, nqu);
        Qu = cheap;
    } else if (n_q <= 0) {
        return -2;
    }
    int t = orc_target_count(T, &p);
    int cs;
    orc_chunk_plan(T, &p, &cs);
    int rcode;
    if (cs < T) rcode = compact_chunked(K, V, Qu, T, nqu, H, d_k, d_v, &p, cs, res);
    else rcode = compact_body(K, V, Qu, T, nqu, H, d_k, d_v, &p, t, res);
    free(cheap);
    return rcode;
}

int orc_kv_compact(const float * K, const float * V, const float * Q, int T, int n_q, int H,
                   int d_k, int d_v, const kv_compact_params * params, kv_compact_result * res) {
    return compact_impl(K, V, Q, T, n_q, H, d_k, d_v, params, res);
}

void orc_result_free(kv_compact_result * r) {
    if (!r) return;
    free(r->selected_indices);
    r->selected_indices = NULL;
    if (r->beta) { free_partial(r->beta, r->n_head_kv); r->beta = NULL; }
    if (r->C_v) { free_partial(r->C_v, r->n_head_kv); r->C_v = NULL; }
    r->t = 0;
    r->n_head_kv = 0;
}

/* api.cpp:980-1111 */
int orc_kv_compact_multi_round(const float * K, const float * V, const float * Q, int T,
                               int n_q, int H, int d_k, int d_v,
                               const kv_compact_params * params, int n_rounds,
                               kv_compact_result * res, kv_compact_stats * per_round) {
    if (!K || !V || !res) return -1;
    if (T <= 0 || H <= 0 || d_k <= 0 || d_v <= 0) return -2;
    if (n_rounds < 1) return -3;
    kv_compact_params pc = params ? *params : orc_params_default();
    if (!Q && !pc.use_cheap_qref) return -1;
    if (Q && n_q <= 0 && !pc.use_cheap_qref) return -2;
    const int ek = H * d_k, ev = H * d_v;
    int * orig = (int *)malloc((size_t)T * sizeof(int));
    for (int i = 0; i < T; i++) orig[i] = i;
    float * cK = (float *)malloc((size_t)T * ek * sizeof(float));
    float * cV = (float *)malloc((size_t)T * ev * sizeof(float));
    memcpy(cK, K, (size_t)T * ek * sizeof(float));
    memcpy(cV, V, (size_t)T * ev * sizeof(float));
    int cT = T;
    float * cheap = NULL;
    const float * Qm = Q;
    int nqm = n_q;
    if (pc.use_cheap_qref || !Q) {
        nqm = cheap_qref_count(T);
        cheap = make_cheap_qref(K, T, ek, nqm);
        Qm = cheap;
    }
    for (int round = 0; round < n_rounds; round++) {
        int nqr = nqm < cT ? nqm : cT;
        kv_compact_result rr;
        memset(&rr, 0, sizeof(rr));
        int rcode = orc_kv_compact(cK, cV, Qm, cT, nqr, H, d_k, d_v, params, &rr);
        if (rcode != 0) {
            orc_result_free(&rr);
            free(orig); free(cK); free(cV); free(cheap);
            return rcode;
        }
        if (per_round) per_round[round] = rr.stats;
        int nT = rr.t;
        int * norig = (int *)malloc((size_t)nT * sizeof(int));
        float * nK = (float *)malloc((size_t)nT * ek * sizeof(float));
        float * nV = (float *)malloc((size_t)nT * ev * sizeof(float));
        for (int j = 0; j < nT; j++) {
            int src = rr.selected_indices[j];
            norig[j] = orig[src];
            memcpy(nK + (size_t)j * ek, cK + (size_t)src * ek, (size_t)ek * sizeof(float));
            for (int h = 0; h < H; h++)
                memcpy(nV + (size_t)j * ev + (size_t)h * d_v, rr.C_v[h] + (size_t)j * d_v,
                       (size_t)d_v * sizeof(float));
        }
        if (round == n_rounds - 1) {
            res->t = nT;
            res->n_head_kv = H;
            res->selected_indices = (int *)malloc((size_t)nT * sizeof(int));
            memcpy(res->selected_indices, norig, (size_t)nT * sizeof(int));
            res->beta = (float **)malloc((size_t)H * sizeof(float *));
            res->C_v = (float **)malloc((size_t)H * sizeof(float *));
            for (int h = 0; h < H; h++) {
                res->beta[h] = (float *)malloc((size_t)nT * sizeof(float));
                memcpy(res->beta[h], rr.beta[h], (size_t)nT * sizeof(float));
                res->C_v[h] = (float *)malloc((size_t)nT * d_v * sizeof(float));
                memcpy(res->C_v[h], rr.C_v[h], (size_t)nT * d_v * sizeof(float));
            }
            res->stats = rr.stats;
        }
        orc_result_free(&rr);
        free(cK); free(cV); free(orig);
        cK = nK; cV = nV; orig = norig; cT = nT;
    }
    orc_quality_stats(K, V, Qm, T, nqm, H, d_k, d_v, res, &res->stats);
    free(orig); free(cK); free(cV); free(cheap);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* codec, state.h:326-629                                                    */
/* ------------------------------------------------------------------------ */

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    uint32_t e = (h >> 10) & 0x1F;
    uint32_t m = h & 0x3FF;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            e = 1;
            while (!(m & 0x400)) { m <<= 1; e--; }
            m &= 0x3FF;
            e = e + (127 - 15);
            bits = sign | (e << 23) | (m << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        e = e + (127 - 15);
        bits = sign | (e << 23) | (m << 13);
    }
    float f; memcpy(&f, &bits, 4);
    return f;
}

/* truncating conversion; NaN maps to Inf, as the reference */
uint16_t orc_f32_to_f16(float val) {
    uint32_t f; memcpy(&f, &val, 4);
    uint32_t sign = (f >> 16) & 0x8000;
    int32_t e = (int32_t)((f >> 23) & 0xFF) - 127 + 15;
    uint32_t m = (f >> 13) & 0x3FF;
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        m = (m | 0x400) >> (1 - e);
        return (uint16_t)(sign | m);
    } else if (e >= 31) {
        return (uint16_t)(sign | 0x7C00);
    }
    return (uint16_t)(sign | ((uint32_t)e << 10) | m);
}

static int block_bytes(int type) {
    if (type == KV_TYPE_F32) return 4;
    if (type == KV_TYPE_F16 || type == KV_TYPE_BF16) return 2;
    if (type == KV_TYPE_Q8_0) return 34;
    if (type == KV_TYPE_Q4_0) return 18;
    if (type == KV_TYPE_Q4_1) return 20;
    return 4;
}

static int is_block_type(int type) {
    return type == KV_TYPE_Q8_0 || type == KV_TYPE_Q4_0 || type == KV_TYPE_Q4_1;
}

int orc_quant_row_elements(int type, size_t row_bytes) {
    if (type == KV_TYPE_F32) return (int)(row_bytes / 4);
    if (type == KV_TYPE_F16 || type == KV_TYPE_BF16) return (int)(row_bytes / 2);
    if (is_block_type(type)) return (int)(row_bytes / (size_t)block_bytes(type)) * 32;
    return (int)(row_bytes / 4);
}

size_t orc_quant_row_bytes(int type, int n) {
    if (type == KV_TYPE_F32) return (size_t)n * 4;
    if (type == KV_TYPE_F16 || type == KV_TYPE_BF16) return (size_t)n * 2;
    if (is_block_type(type)) return (size_t)(n / 32) * (size_t)block_bytes(type);
    return (size_t)n * 4;
}

static void convert_to_f32(const uint8_t * src, int type, float * dst, size_t n) {
    if (type == KV_TYPE_F32) {
        memcpy(dst, src, n * sizeof(float));
    } else if (type == KV_TYPE_F16) {
        for (size_t i = 0; i < n; i++) {
            uint16_t h; memcpy(&h, src + 2 * i, 2);
            dst[i] = orc_f16_to_f32(h);
        }
    } else if (type == KV_TYPE_BF16) {
        /* extension type (no reference counterpart): exact up-cast */
        for (size_t i = 0; i < n; i++) {
            uint16_t h; memcpy(&h, src + 2 * i, 2);
            uint32_t u = (uint32_t)h << 16;
            memcpy(dst + i, &u, 4);
        }
    } else if (type == KV_TYPE_Q8_0) {
        for (size_t b = 0; b < n / 32; b++) {
            const uint8_t * s = src + b * 34;
            uint16_t h; memcpy(&h, s, 2);
            float d = orc_f16_to_f32(h);
            for (int i = 0; i < 32; i++) dst[b * 32 + i] = d * (float)(int8_t)s[2 + i];
        }
    } else if (type == KV_TYPE_Q4_0) {
        for (size_t b = 0; b < n / 32; b++) {
            const uint8_t * s = src + b * 18;
            uint16_t h; memcpy(&h, s, 2);
            float d = orc_f16_to_f32(h);
            for (int i = 0; i < 16; i++) {
                dst[b * 32 + 2 * i] = d * ((float)(s[2 + i] & 0xF) - 8.0f);
                dst[b * 32 + 2 * i + 1] = d * ((float)(s[2 + i] >> 4) - 8.0f);
            }
        }
    } else if (type == KV_TYPE_Q4_1) {
        for (size_t b = 0; b < n / 32; b++) {
            const uint8_t * s = src + b * 20;
            uint16_t hd, hm; memcpy(&hd, s, 2); memcpy(&hm, s + 2, 2);
            float d = orc_f16_to_f32(hd), m = orc_f16_to_f32(hm);
            for (int i = 0; i < 16; i++) {
                dst[b * 32 + 2 * i] = d * (float)(s[4 + i] & 0xF) + m;
                dst[b * 32 + 2 * i + 1] = d * (float)(s[4 + i] >> 4) + m;
            }
        }
    } else {
        memset(dst, 0, n * sizeof(float));
    }
}

static inline float fmax_ref(float a, float b) { return (a < b) ? b : a; }  /* std::max */
static inline float fmin_ref(float a, float b) { return (b < a) ? b : a; }  /* std::min */

size_t orc_quantize_row(const float * src, int type, int n, uint8_t * dst) {
    if (type == KV_TYPE_F32) {
        memcpy(dst, src, (size_t)n * sizeof(float));
        return (size_t)n * sizeof(float);
    }
    if (type == KV_TYPE_F16) {
        for (int i = 0; i < n; i++) {
            uint16_t h = orc_f32_to_f16(src[i]);
            memcpy(dst + 2 * i, &h, 2);
        }
        return (size_t)n * 2;
    }
    if (type == KV_TYPE_BF16) {
        /* round to nearest, ties to even; NaN -> quiet NaN */
        for (int i = 0; i < n; i++) {
            uint32_t u; memcpy(&u, src + i, 4);
            uint16_t h = ((u & 0x7fffffffu) > 0x7f800000u) ? (uint16_t)((u >> 16) | 0x40u)
                                                          : (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
            memcpy(dst + 2 * i, &h, 2);
        }
        return (size_t)n * 2;
    }
    int nb = n / 32;
    if (type == KV_TYPE_Q8_0) {
        for (int b = 0; b < nb; b++) {
            const float * x = src + b * 32;
            uint8_t * o = dst + (size_t)b * 34;
            float amax = 0.0f;
            for (int i = 0; i < 32; i++) { float a = fabsf(x[i]); if (a > amax) amax = a; }
            float d = amax / 127.0f;
            uint16_t h = orc_f32_to_f16(d);
            memcpy(o, &h, 2);
            float id = (d != 0.0f) ? 127.0f / amax : 0.0f;
            for (int i = 0; i < 32; i++) {
                float v = x[i] * id;
                o[2 + i] = (uint8_t)(int8_t)roundf(fmax_ref(-128.0f, fmin_ref(127.0f, v)));
            }
        }
        return (size_t)nb * 34;
    }
    if (type == KV_TYPE_Q4_0) {
        for (int b = 0; b < nb; b++) {
            const float * x = src + b * 32;
            uint8_t * o = dst + (size_t)b * 18;
            float amax = 0.0f;
            for (int i = 0; i < 32; i++) { float a = fabsf(x[i]); if (a > amax) amax = a; }
            float d = amax / 7.0f;
            uint16_t h = orc_f32_to_f16(d);
            memcpy(o, &h, 2);
            float id = (d != 0.0f) ? 7.0f / amax : 0.0f;
            for (int i = 0; i < 16; i++) {
                float v0 = x[2 * i] * id + 8.0f;
                float v1 = x[2 * i + 1] * id + 8.0f;
                uint8_t q0 = (uint8_t)fmax_ref(0.0f, fmin_ref(15.0f, roundf(v0)));
                uint8_t q1 = (uint8_t)fmax_ref(0.0f, fmin_ref(15.0f, roundf(v1)));
                o[2 + i] = (uint8_t)(q0 | (q1 << 4));
            }
        }
        return (size_t)nb * 18;
    }
    if (type == KV_TYPE_Q4_1) {
        for (int b = 0; b < nb; b++) {
            const float * x = src + b * 32;
            uint8_t * o = dst + (size_t)b * 20;
            float mn = x[0], mx = x[0];
            for (int i = 1; i < 32; i++) { if (x[i] < mn) mn = x[i]; if (x[i] > mx) mx = x[i]; }
            float d = (mx - mn) / 15.0f;
            uint16_t hd = orc_f32_to_f16(d), hm = orc_f32_to_f16(mn);
            memcpy(o, &hd, 2);
            memcpy(o + 2, &hm, 2);
            float id = (d != 0.0f) ? 15.0f / (mx - mn) : 0.0f;
            for (int i = 0; i < 16; i++) {
                float v0 = (x[2 * i] - mn) * id;
                float v1 = (x[2 * i + 1] - mn) * id;
                uint8_t q0 = (uint8_t)fmax_ref(0.0f, fmin_ref(15.0f, roundf(v0)));
                uint8_t q1 = (uint8_t)fmax_ref(0.0f, fmin_ref(15.0f, roundf(v1)));
                o[4 + i] = (uint8_t)(q0 | (q1 << 4));
            }
        }
        return (size_t)nb * 20;
    }
    return 0;
}

int orc_dequantize_row(const uint8_t * src, int type, size_t row_bytes, float * dst, int max_el) {
    int n = orc_quant_row_elements(type, row_bytes);
    if (n > max_el) n = max_el;
    convert_to_f32(src, type, dst, (size_t)n);
    return n;
}

/* api.cpp:1182-1257 */
int orc_kv_compact_quantized(const uint8_t * Kq, const uint8_t * Vq, const float * Q,
                             int k_type, int v_type, size_t k_rb, size_t v_rb,
                             int T, int n_q, int H, int d_k, int d_v,
                             const kv_compact_params * params, kv_compact_quant_result * res) {
    if (!Kq || !Vq || !res) return -1;
    if (T <= 0 || H <= 0 || d_k <= 0 || d_v <= 0) return -2;
    const int ek = H * d_k, ev = H * d_v;
    if (orc_quant_row_elements(k_type, k_rb) != ek || orc_quant_row_elements(v_type, v_rb) != ev)
        return -4;
    float * Kf = (float *)malloc((size_t)T * ek * sizeof(float));
    float * Vf = (float *)malloc((size_t)T * ev * sizeof(float));
    for (int i = 0; i < T; i++) {
        convert_to_f32(Kq + (size_t)i * k_rb, k_type, Kf + (size_t)i * ek, (size_t)ek);
        convert_to_f32(Vq + (size_t)i * v_rb, v_type, Vf + (size_t)i * ev, (size_t)ev);
    }
    memset(&res->base, 0, sizeof(res->base));
    int rcode = orc_kv_compact(Kf, Vf, Q, T, n_q, H, d_k, d_v, params, &res->base);
    if (rcode != 0) { free(Kf); free(Vf); return rcode; }
    int t = res->base.t;
    res->k_type = k_type;
    res->v_type = v_type;
    res->k_row_bytes = k_rb;
    res->v_row_bytes = v_rb;
    res->K_out = (uint8_t *)malloc((size_t)t * k_rb);
    res->V_out = (uint8_t *)malloc((size_t)t * v_rb);
    for (int j = 0; j < t; j++)
        orc_quantize_row(Kf + (size_t)res->base.selected_indices[j] * ek, k_type, ek,
                         res->K_out + (size_t)j * k_rb);
    float * vrow = (float *)malloc((size_t)ev * sizeof(float));
    for (int j = 0; j < t; j++) {
        for (int h = 0; h < H; h++)
            memcpy(vrow + (size_t)h * d_v, res->base.C_v[h] + (size_t)j * d_v, (size_t)d_v * sizeof(float));
        orc_quantize_row(vrow, v_type, ev, res->V_out + (size_t)j * v_rb);
    }
    free(vrow); free(Kf); free(Vf);
    return 0;
}

void orc_quant_result_free(kv_compact_quant_result * r) {
    if (!r) return;
    orc_result_free(&r->base);
    free(r->K_out); r->K_out = NULL;
    free(r->V_out); r->V_out = NULL;
}

/* ------------------------------------------------------------------------ */
/* llama.cpp state blob: parse (state.h:104-222), the CLI's cross-layer      */
/* selection and refit (kv-compact.cpp:380-690), and the compacted blob      */
/* (build_compacted_state, state.h:645-810).                                 */
/* ------------------------------------------------------------------------ */

typedef struct {
    int32_t k_type, v_type;
    uint64_t k_size_row, v_size_row;
    uint32_t v_size_el, n_embd_v_hdr;
    int nk, nv;                /* elements per K / V row (V: [cell][nv] after the transpose) */
    float * K;                 /* [cell][nk] */
    float * V;                 /* [cell][nv] */
} orc_layer;

typedef struct {
    uint32_t n_stream, cell_count, v_trans, n_layer;
    int32_t * pos;             /* [cell] */
    int32_t * ext;             /* [cell][2] (n_pos_per_embd > 1) */
    uint32_t * n_seq;          /* [cell] */
    int32_t ** seq;            /* [cell][n_seq] */
    orc_layer * layers;
    size_t kv_end;             /* offset of the trailing bytes */
} orc_state;

static void orc_state_release(orc_state * s) {
    if (s->seq)
        for (uint32_t c = 0; c < s->cell_count; c++) free(s->seq[c]);
    if (s->layers)
        for (uint32_t l = 0; l < s->n_layer; l++) { free(s->layers[l].K); free(s->layers[l].V); }
    free(s->pos); free(s->ext); free(s->n_seq); free(s->seq); free(s->layers);
    memset(s, 0, sizeof(*s));
}

static int rd(const uint8_t ** p, const uint8_t * end, void * v, size_t n) {
    if ((size_t)(end - *p) < n) return 0;
    memcpy(v, *p, n);
    *p += n;
    return 1;
}

/* parsed_kv_state::parse (state.h:104-222). Returns 1 on success. Streams
 * after the first must be empty (only stream 0 is kept here); a non-empty one
 * sets *extra_streams. */
static int orc_state_parse(const uint8_t * data, size_t size, uint32_t n_pos, orc_state * s, int * extra_streams) {
    const uint8_t * p = data;
    const uint8_t * end = data + size;
    memset(s, 0, sizeof(*s));
    *extra_streams = 0;
    if (!rd(&p, end, &s->n_stream, 4)) return 0;
    for (uint32_t st = 0; st < s->n_stream; st++) {
        uint32_t cc;
        if (!rd(&p, end, &cc, 4)) return 0;
        if (cc == 0) continue;
        if (st > 0) { *extra_streams = 1; return 1; }   /* only stream 0 may hold cells */
        /* a record takes at least 8 bytes: larger counts are malformed (the
         * reference would size its cell table first and fail while reading) */
        if (cc > (size_t)(end - p) / 8) return 0;
        s->cell_count = cc;
        s->pos = (int32_t *)calloc(cc, 4);
        s->ext = (int32_t *)calloc((size_t)cc * 2, 4);
        s->n_seq = (uint32_t *)calloc(cc, 4);
        s->seq = (int32_t **)calloc(cc, sizeof(int32_t *));
        for (uint32_t c = 0; c < cc; c++) {
            if (!rd(&p, end, &s->pos[c], 4)) return 0;
            if (!rd(&p, end, &s->n_seq[c], 4)) return 0;
            if (n_pos > 1) {
                if (!rd(&p, end, &s->ext[2 * c], 4)) return 0;
                if (!rd(&p, end, &s->ext[2 * c + 1], 4)) return 0;
            }
            /* each id needs 4 bytes: a count beyond the blob fails below */
            if ((size_t)(end - p) / 4 < s->n_seq[c]) return 0;
            s->seq[c] = (int32_t *)malloc((size_t)(s->n_seq[c] ? s->n_seq[c] : 1) * 4);
            for (uint32_t i = 0; i < s->n_seq[c]; i++)
                if (!rd(&p, end, &s->seq[c][i], 4)) return 0;
        }
        if (!rd(&p, end, &s->v_trans, 4)) return 0;
        if (!rd(&p, end, &s->n_layer, 4)) return 0;
        if (s->n_layer > (size_t)(end - p) / 24) return 0;   /* two headers of >= 12 bytes per layer */
        s->layers = (orc_layer *)calloc(s->n_layer ? s->n_layer : 1, sizeof(orc_layer));
        for (uint32_t l = 0; l < s->n_layer; l++) {
            orc_layer * ld = &s->layers[l];
            if (!rd(&p, end, &ld->k_type, 4)) return 0;
            if (!rd(&p, end, &ld->k_size_row, 8)) return 0;
            const uint64_t bytes = (uint64_t)cc * ld->k_size_row;
            if ((uint64_t)(end - p) < bytes) return 0;
            ld->nk = orc_quant_row_elements(ld->k_type, (size_t)ld->k_size_row);
            ld->K = (float *)malloc(((size_t)cc * ld->nk + 1) * sizeof(float));
            for (uint32_t c = 0; c < cc; c++)
                convert_to_f32(p + (size_t)c * ld->k_size_row, ld->k_type, ld->K + (size_t)c * ld->nk, (size_t)ld->nk);
            p += bytes;
        }
        for (uint32_t l = 0; l < s->n_layer; l++) {
            orc_layer * ld = &s->layers[l];
            if (!rd(&p, end, &ld->v_type, 4)) return 0;
            if (!s->v_trans) {
                if (!rd(&p, end, &ld->v_size_row, 8)) return 0;
                const uint64_t bytes = (uint64_t)cc * ld->v_size_row;
                if ((uint64_t)(end - p) < bytes) return 0;
                ld->nv = orc_quant_row_elements(ld->v_type, (size_t)ld->v_size_row);
                ld->V = (float *)malloc(((size_t)cc * ld->nv + 1) * sizeof(float));
                for (uint32_t c = 0; c < cc; c++)
                    convert_to_f32(p + (size_t)c * ld->v_size_row, ld->v_type, ld->V + (size_t)c * ld->nv,
                                   (size_t)ld->nv);
                p += bytes;
            } else {
                /* [embd][cell] storage: decoded as one flat run of
                 * n_embd * cell values, then transposed (state.h:425-462) */
                if (!rd(&p, end, &ld->v_size_el, 4)) return 0;
                if (!rd(&p, end, &ld->n_embd_v_hdr, 4)) return 0;
                const uint64_t bytes = (uint64_t)ld->n_embd_v_hdr * cc * ld->v_size_el;
                if ((uint64_t)(end - p) < bytes) return 0;
                const size_t n = (size_t)ld->n_embd_v_hdr * cc;
                /* the flat decode must stay inside the section (a smaller
                 * v_size_el would make the reference read past it) */
                if (orc_quant_row_bytes(ld->v_type, (int)n) > bytes) return 0;
                ld->nv = (int)ld->n_embd_v_hdr;
                float * tmp = (float *)calloc(n + 1, sizeof(float));
                convert_to_f32(p, ld->v_type, tmp, n);
                ld->V = (float *)malloc((n + 1) * sizeof(float));
                for (uint32_t d = 0; d < ld->n_embd_v_hdr; d++)
                    for (uint32_t c = 0; c < cc; c++) ld->V[(size_t)c * ld->nv + d] = tmp[(size_t)d * cc + c];
                free(tmp);
                p += bytes;
            }
        }
    }
    s->kv_end = (size_t)(p - data);
    return 1;
}

int orc_state_parse_info(const uint8_t * blob, size_t size, uint32_t n_pos, kvc_state_info * info) {
    if (!blob || !info) return -1;
    orc_state s;
    int extra = 0;
    if (!orc_state_parse(blob, size, n_pos, &s, &extra)) { orc_state_release(&s); return -2; }
    memset(info, 0, sizeof(*info));
    if (extra) { orc_state_release(&s); return KV_COMPACT_E_UNSUPPORTED; }
    info->n_stream = s.n_stream;
    info->cell_count = s.cell_count;
    info->v_trans = s.v_trans;
    info->n_layer = s.n_layer;
    if (s.n_layer > 0) { info->n_embd_k = s.layers[0].nk; info->n_embd_v = s.layers[0].nv; }
    info->kv_bytes = s.kv_end;
    info->trailing_bytes = size - s.kv_end;
    orc_state_release(&s);
    return 0;
}

typedef struct { uint8_t * p; size_t n, cap; } orc_buf;

static void put(orc_buf * b, const void * v, size_t n) {
    if (b->n + n > b->cap) {
        size_t c = b->cap ? b->cap : 4096;
        while (c < b->n + n) c *= 2;
        b->p = (uint8_t *)realloc(b->p, c);
        b->cap = c;
    }
    memcpy(b->p + b->n, v, n);
    b->n += n;
}

static int state_type_ok(int32_t t) {
    return t == KV_TYPE_F32 || t == KV_TYPE_F16 || t == KV_TYPE_Q8_0 || t == KV_TYPE_Q4_0 || t == KV_TYPE_Q4_1;
}

/* The CLI's compaction of stream 0 (kv-compact.cpp:380-690) and the blob
 * writer (state.h:645-810). beta is 0 for every kept cell (the CLI never fits
 * it, kv-compact.cpp:611) but the writer still adds (beta * sqrtf(d_k)) *
 * direction to each kept key, so the directions are computed. */
int orc_state_compact(const uint8_t * blob, size_t size, const kvc_state_params * sp,
                      uint8_t ** out, size_t * out_size, int32_t * sel_out) {
    if (!blob || !sp || !out || !out_size) return -1;
    orc_state s;
    int extra = 0;
    if (!orc_state_parse(blob, size, sp->n_pos_per_embd, &s, &extra)) { orc_state_release(&s); return -2; }
    if (extra) { orc_state_release(&s); return KV_COMPACT_E_UNSUPPORTED; }
    if (s.cell_count == 0 || s.n_layer == 0) { orc_state_release(&s); return -2; }
    const int T = (int)s.cell_count, L = (int)s.n_layer, H = sp->n_head_kv;
    const int nk = s.layers[0].nk, nv = s.layers[0].nv;
    if (H <= 0 || nk <= 0 || nv <= 0 || nk % H || nv % H) { orc_state_release(&s); return -2; }
    for (int l = 0; l < L; l++) {
        const orc_layer * ld = &s.layers[l];
        if (!state_type_ok(ld->k_type) || !state_type_ok(ld->v_type) || ld->nk != nk || ld->nv != nv) {
            orc_state_release(&s);
            return KV_COMPACT_E_UNSUPPORTED;
        }
    }
    const int dk = nk / H, dv = nv / H;
    int t = (int)(T * sp->compact_ratio);   /* kv-compact.cpp:269 */
    if (t < 1) t = 1;
    int nq = sp->n_ref_queries;             /* kv-compact.cpp:274-277 */
    if (nq <= 0) nq = T / 4 > 16 ? T / 4 : 16;
    if (nq > T) nq = T;
    if (t > T) { orc_state_release(&s); return -2; }
    if (nq > 8192) { orc_state_release(&s); return KV_COMPACT_E_UNSUPPORTED; }
    const int ref_start = T - nq;
    const float inv_sqrt = 1.0f / sqrtf((float)dk);
    unsigned char * on = (unsigned char *)malloc((size_t)L);
    for (int l = 0; l < L; l++) on[l] = sp->layer_filter ? (sp->layer_filter(l, L, sp->layer_filter_data) != 0) : 1;

    /* scores, softmax and importance per (layer, head); global importance as
     * the max over all of them (0 start) or the sensitivity-weighted sum in
     * (layer, head) order (kv-compact.cpp:500-571) */
    float * S = (float *)malloc((size_t)L * H * nq * T * sizeof(float));
    float * A = (float *)malloc((size_t)L * H * nq * T * sizeof(float));
    float * himp = (float *)malloc((size_t)L * H * T * sizeof(float));
    float * sens = (float *)malloc((size_t)L * H * sizeof(float));
    float * gimp = (float *)calloc((size_t)T, sizeof(float));
    int n_heads = 0;
    for (int l = 0; l < L; l++) {
        if (!on[l]) continue;
        const float * K = s.layers[l].K;
        for (int h = 0; h < H; h++) {
            const size_t o = ((size_t)l * H + h) * nq * T;
            float * ih = himp + (size_t)n_heads * T;
            orc_scores(K + (size_t)ref_start * nk + (size_t)h * dk, K + (size_t)h * dk, S + o, nq, T, dk, nk, nk,
                       inv_sqrt);
            orc_softmax_importance(S + o, A + o, ih, NULL, NULL, nq, T, 0);
            if (sp->sensitivity_budget) sens[n_heads] = orc_head_sensitivity(A + o, nq, T);
            else for (int j = 0; j < T; j++) if (ih[j] > gimp[j]) gimp[j] = ih[j];
            n_heads++;
        }
    }
    if (sp->sensitivity_budget)
        for (int k = 0; k < n_heads; k++)
            for (int j = 0; j < T; j++) gimp[j] += sens[k] * himp[(size_t)k * T + j];
    int * sel = (int *)malloc((size_t)t * sizeof(int));
    orc_select_topk(gimp, T, t, 0, sel);   /* partial_sort + sort, kv-compact.cpp:573-582 */
    if (sel_out) for (int j = 0; j < t; j++) sel_out[j] = sel[j];

    /* values (kv-compact.cpp:594-635) and beta directions (kv-compact.cpp:659-685) */
    float * cv = (float *)malloc((size_t)L * H * t * dv * sizeof(float));
    float * dir = (float *)calloc((size_t)L * H * dk, sizeof(float));
    float * X = (float *)malloc((size_t)nq * t * sizeof(float));
    float * Y = (float *)malloc((size_t)nq * dv * sizeof(float));
    float * Qh = (float *)malloc((size_t)nq * dk * sizeof(float));
    float * ones = (float *)malloc((size_t)nq * sizeof(float));
    for (int i = 0; i < nq; i++) ones[i] = 1.0f;
    for (int l = 0; l < L; l++) {
        const orc_layer * ld = &s.layers[l];
        for (int h = 0; h < H; h++) {
            float * c = cv + ((size_t)l * H + h) * t * dv;
            if (!on[l]) {
                for (int j = 0; j < t; j++)
                    memcpy(c + (size_t)j * dv, ld->V + (size_t)sel[j] * nv + (size_t)h * dv, (size_t)dv * 4);
                continue;
            }
            const size_t o = ((size_t)l * H + h) * nq * T;
            for (int i = 0; i < nq; i++)
                for (int j = 0; j < t; j++) X[(size_t)i * t + j] = S[o + (size_t)i * T + sel[j]] + 0.0f;
            orc_softmax_rows(X, nq, t);
            for (int i = 0; i < nq; i++)
                for (int e = 0; e < dv; e++) {
                    float acc = 0.0f;
                    for (int j = 0; j < T; j++)
                        acc += A[o + (size_t)i * T + j] * ld->V[(size_t)j * nv + (size_t)h * dv + e];
                    Y[(size_t)i * dv + e] = acc;
                }
            orc_ls_solve(X, Y, c, nq, t, dv, 1e-6f);
            for (int i = 0; i < nq; i++)
                memcpy(Qh + (size_t)i * dk, ld->K + (size_t)(ref_start + i) * nk + (size_t)h * dk, (size_t)dk * 4);
            orc_ls_solve(Qh, ones, dir + ((size_t)l * H + h) * dk, nq, dk, 1, 1e-6f);
        }
    }

    /* the compacted blob, state.h:645-810 */
    orc_buf b = {0};
    put(&b, &s.n_stream, 4);
    const uint32_t tc = (uint32_t)t;
    put(&b, &tc, 4);
    for (int j = 0; j < t; j++) {
        const int c = sel[j];
        put(&b, &s.pos[c], 4);
        put(&b, &s.n_seq[c], 4);
        if (sp->n_pos_per_embd > 1) put(&b, &s.ext[2 * c], 8);
        put(&b, s.seq[c], (size_t)s.n_seq[c] * 4);
    }
    put(&b, &s.v_trans, 4);
    put(&b, &s.n_layer, 4);
    const float scale = sqrtf((float)dk);
    float * row = (float *)malloc((size_t)(nk > nv ? nk : nv) * sizeof(float) + 4);
    uint8_t * rb = (uint8_t *)malloc((size_t)(nk > nv ? nk : nv) * 4 + (size_t)t * 4 + 64);
    for (int l = 0; l < L; l++) {
        const orc_layer * ld = &s.layers[l];
        put(&b, &ld->k_type, 4);
        put(&b, &ld->k_size_row, 8);
        for (int j = 0; j < t; j++) {
            memcpy(row, ld->K + (size_t)sel[j] * nk, (size_t)nk * 4);
            for (int h = 0; h < H; h++) {
                const float bs = 0.0f * scale;
                const float * dh = dir + ((size_t)l * H + h) * dk;
                for (int d = 0; d < dk; d++) row[h * dk + d] += bs * dh[d];
            }
            put(&b, rb, orc_quantize_row(row, ld->k_type, nk, rb));
        }
    }
    for (int l = 0; l < L; l++) {
        const orc_layer * ld = &s.layers[l];
        put(&b, &ld->v_type, 4);
        if (!s.v_trans) {
            put(&b, &ld->v_size_row, 8);
            for (int j = 0; j < t; j++) {
                for (int h = 0; h < H; h++)
                    memcpy(row + (size_t)h * dv, cv + (((size_t)l * H + h) * t + j) * dv, (size_t)dv * 4);
                put(&b, rb, orc_quantize_row(row, ld->v_type, nv, rb));
            }
        } else {
            put(&b, &ld->v_size_el, 4);
            const uint32_t ne = (uint32_t)(H * dv);
            put(&b, &ne, 4);
            float * col = (float *)malloc((size_t)t * sizeof(float));
            for (uint32_t d = 0; d < ne; d++) {
                const int h = (int)d / dv, e = (int)d % dv;
                for (int j = 0; j < t; j++) col[j] = cv[(((size_t)l * H + h) * t + j) * dv + e];
                if (ld->v_type == KV_TYPE_F32 || ld->v_type == KV_TYPE_F16 || ld->v_type == KV_TYPE_Q8_0 ||
                    ld->v_type == KV_TYPE_Q4_0 || ld->v_type == KV_TYPE_Q4_1)
                    put(&b, rb, orc_quantize_row(col, ld->v_type, t, rb));
            }
            free(col);
        }
    }
    const uint32_t zero = 0;   /* the other (empty) streams */
    for (uint32_t st = 1; st < s.n_stream; st++) put(&b, &zero, 4);
    if (size > s.kv_end) put(&b, blob + s.kv_end, size - s.kv_end);
    *out = b.p;
    *out_size = b.n;
    free(row); free(rb); free(on); free(S); free(A); free(himp); free(sens); free(gimp); free(sel);
    free(cv); free(dir); free(X); free(Y); free(Qh); free(ones);
    orc_state_release(&s);
    return 0;
}

void orc_state_free(uint8_t * p) { free(p); }
