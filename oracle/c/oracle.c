/* CPU oracle for the screened DF-J path -- TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Every function restates the reference's algorithm in its own operation order where the
 * reference fixes one (3x3 cofactor expansions, pair-quantity sequence, metric formula), citing
 * the reference file:line it follows. Transcendentals are glibc's (exp, sqrt, pow, erf), so the
 * oracle shares no arithmetic code with the HIP library it checks.
 *
 * One deliberate restatement: the (iso aux | full-covariance pair) node sum of
 * gs_dft/coulomb/ri.py:167-185 is written with the rotation invariants of the pair precision
 * (I1 = tr, I2 = sum of principal 2x2 minors, I3 = det) instead of an eigendecomposition.
 * Cayley-Hamilton makes the two identical: with a = beta + t^2 and c = t^2 beta,
 *   prod_k Gamma_k = a^3 I3 + a^2 c I2 + a c^2 I1 + c^3,
 *   sum_k W_k prod_{j!=k} Gamma_j = beta (a^2 I3 q0 + a c (I1 q1 - q2) + c^2 q1),
 * with q0 = |d|^2, q1 = d.A d, q2 = |A d|^2. The tests pin this against a literal eigh-based
 * restatement of the reference kernel.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define NQ 20

static const double PI15 = 5.568327996831708;        /* math.pi ** 1.5 */

/* The worker count of the OpenMP loops (1 when built without OpenMP). */
int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ---------------------------------------------------------------- quadrature table */

void orc_quad_table(int n, double* t, double* w) {
    /* Roots of P_n by Newton from the Tricomi initial guess, ascending; then the half-line map
     * t = s/(1-s), s = (x+1)/2, w_t = (w/2)/(1-s)^2 of gs_dft/integrals/dense.py:46-53. */
    for (int i = 0; i < n; ++i) {
        double x = -cos(M_PI * (i + 0.75) / (n + 0.5));
        double dp = 1.0;
        for (int it = 0; it < 100; ++it) {
            double p0 = 1.0, p1 = x;
            for (int k = 2; k <= n; ++k) {
                double p2 = ((2.0 * k - 1.0) * x * p1 - (k - 1.0) * p0) / k;
                p0 = p1;
                p1 = p2;
            }
            dp = n * (x * p1 - p0) / (x * x - 1.0);
            double dx = p1 / dp;
            x -= dx;
            if (fabs(dx) < 1e-17) break;
        }
        {   /* final derivative at the converged root */
            double p0 = 1.0, p1 = x;
            for (int k = 2; k <= n; ++k) {
                double p2 = ((2.0 * k - 1.0) * x * p1 - (k - 1.0) * p0) / k;
                p0 = p1;
                p1 = p2;
            }
            dp = n * (x * p1 - p0) / (x * x - 1.0);
        }
        double wl = 2.0 / ((1.0 - x * x) * dp * dp);
        double s = (x + 1.0) / 2.0;
        t[i] = s / (1.0 - s);
        w[i] = (wl / 2.0) * (1.0 / ((1.0 - s) * (1.0 - s)));
    }
}

/* The node table every three-centre routine uses: Newton-derived by default, replaceable by the
 * caller (the tests install numpy's leggauss table, which is the reference's own). */
static double g_tq[NQ], g_wq[NQ];
static int g_table_set = 0;

void orc_set_quad_table(const double* t, const double* w) {
    memcpy(g_tq, t, sizeof g_tq);
    memcpy(g_wq, w, sizeof g_wq);
    g_table_set = 1;
}

static void node_table(double* t, double* w) {
    if (!g_table_set) {
        orc_quad_table(NQ, g_tq, g_wq);
        g_table_set = 1;
    }
    memcpy(t, g_tq, sizeof g_tq);
    memcpy(w, g_wq, sizeof g_wq);
}

/* ---------------------------------------------------------------- 3x3 algebra */

/* gs_dft/integrals/linalg3.py:17-22 */
static double det3(const double* A) {
    return A[0] * (A[4] * A[8] - A[5] * A[7])
         - A[1] * (A[3] * A[8] - A[5] * A[6])
         + A[2] * (A[3] * A[7] - A[4] * A[6]);
}

/* gs_dft/integrals/linalg3.py:26-41 */
static void adj3(const double* A, double* c) {
    c[0] = A[4] * A[8] - A[5] * A[7];
    c[1] = A[2] * A[7] - A[1] * A[8];
    c[2] = A[1] * A[5] - A[2] * A[4];
    c[3] = A[5] * A[6] - A[3] * A[8];
    c[4] = A[0] * A[8] - A[2] * A[6];
    c[5] = A[2] * A[3] - A[0] * A[5];
    c[6] = A[3] * A[7] - A[4] * A[6];
    c[7] = A[1] * A[6] - A[0] * A[7];
    c[8] = A[0] * A[4] - A[1] * A[3];
}

static void matvec3(const double* A, const double* x, double* y) {
    for (int k = 0; k < 3; ++k) y[k] = A[3 * k] * x[0] + A[3 * k + 1] * x[1] + A[3 * k + 2] * x[2];
}

/* gs_dft/integrals/linalg3.py:49-51: adj(A) b / det(A) */
static void solve3(const double* A, const double* b, double* x) {
    double c[9];
    adj3(A, c);
    double det = det3(A);
    for (int k = 0; k < 3; ++k) x[k] = (c[3 * k] * b[0] + c[3 * k + 1] * b[1] + c[3 * k + 2] * b[2]) / det;
}

/* ---------------------------------------------------------------- chart */

/* gs_dft/basis/spectral.py:33-40 */
static void quat_rotation(const double* q, double* R, double* qn, double* nrm_out) {
    double nrm = sqrt(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]);
    double den = nrm + 1e-12;
    double w = q[0] / den, x = q[1] / den, y = q[2] / den, z = q[3] / den;
    R[0] = 1 - 2 * (y * y + z * z); R[1] = 2 * (x * y - w * z); R[2] = 2 * (x * z + w * y);
    R[3] = 2 * (x * y + w * z); R[4] = 1 - 2 * (x * x + z * z); R[5] = 2 * (y * z - w * x);
    R[6] = 2 * (x * z - w * y); R[7] = 2 * (y * z + w * x); R[8] = 1 - 2 * (x * x + y * y);
    if (qn) { qn[0] = w; qn[1] = x; qn[2] = y; qn[3] = z; }
    if (nrm_out) *nrm_out = nrm;
}

/* gs_dft/basis/spectral.py:72-82. A_ik = sum_j (R_ij a_j) R_kj, evaluated for i <= k and mirrored
 * so the stored precision is exactly symmetric. */
void orc_chart(int64_t M, const double* quat, const double* log_scale, double* A9, double* norm) {
    for (int64_t m = 0; m < M; ++m) {
        double R[9];
        quat_rotation(quat + 4 * m, R, NULL, NULL);
        const double* l = log_scale + 3 * m;
        double a[3] = {exp(l[0]), exp(l[1]), exp(l[2])};
        double* A = A9 + 9 * m;
        for (int i = 0; i < 3; ++i)
            for (int k = i; k < 3; ++k) {
                double v = (R[3 * i] * a[0]) * R[3 * k] + (R[3 * i + 1] * a[1]) * R[3 * k + 1]
                         + (R[3 * i + 2] * a[2]) * R[3 * k + 2];
                A[3 * i + k] = v;
                A[3 * k + i] = v;
            }
        double detA = exp(l[0] + l[1] + l[2]);
        norm[m] = pow(8.0 * detA / (M_PI * M_PI * M_PI), 0.25);
    }
}

/* ---------------------------------------------------------------- pair quantities */

/* gs_dft/coulomb/stream.py:203-215 for one pair; also returns det(Ah). */
static void pair_q(const double* Ai, const double* Aj, const double* mui, const double* muj,
                   double Ni, double Nj, double* Ah, double* Pc, double* KN, double* det_out) {
    for (int k = 0; k < 9; ++k) Ah[k] = Ai[k] + Aj[k];
    double r1[3], r2[3], rhs[3];
    matvec3(Ai, mui, r1);
    matvec3(Aj, muj, r2);
    for (int k = 0; k < 3; ++k) rhs[k] = r1[k] + r2[k];
    solve3(Ah, rhs, Pc);
    double d[3] = {mui[0] - muj[0], mui[1] - muj[1], mui[2] - muj[2]};
    double Ajd[3], x[3], z[3];
    matvec3(Aj, d, Ajd);
    solve3(Ah, Ajd, x);
    matvec3(Ai, x, z);
    double e = d[0] * z[0] + d[1] * z[1] + d[2] * z[2];
    double K = exp(-e);
    *KN = Ni * Nj * K;
    if (det_out) *det_out = det3(Ah);
}

void orc_pair_quantities(int64_t M, const double* A9, const double* mu, const double* norm,
                         int64_t n, const int32_t* pi, const int32_t* pj,
                         double* Ah9, double* Pc, double* KN) {
    (void)M;
    for (int64_t a = 0; a < n; ++a) {
        int i = pi[a], j = pj[a];
        pair_q(A9 + 9 * i, A9 + 9 * j, mu + 3 * i, mu + 3 * j, norm[i], norm[j],
               Ah9 + 9 * a, Pc + 3 * a, KN + a, NULL);
    }
}

/* gs_dft/screening/pairs.py:342-345: S = KN pi^1.5 / sqrt(det3(Ah)). */
static double overlap_one(const double* A9, const double* mu, const double* norm, int i, int j) {
    double Ah[9], Pc[3], KN, det;
    pair_q(A9 + 9 * i, A9 + 9 * j, mu + 3 * i, mu + 3 * j, norm[i], norm[j], Ah, Pc, &KN, &det);
    return KN * PI15 / sqrt(det);
}

typedef struct { double* A9; double* norm; } Chart;

static Chart chart_alloc(int64_t M, const double* quat, const double* log_scale) {
    Chart c;
    c.A9 = (double*)malloc(sizeof(double) * 9 * (M > 0 ? M : 1));
    c.norm = (double*)malloc(sizeof(double) * (M > 0 ? M : 1));
    orc_chart(M, quat, log_scale, c.A9, c.norm);
    return c;
}

static void chart_free(Chart* c) { free(c->A9); free(c->norm); }

void orc_overlap_pairs(int64_t M, const double* quat, const double* log_scale,
                       const double* centers, int64_t n, const int32_t* pi, const int32_t* pj,
                       double* S) {
    Chart c = chart_alloc(M, quat, log_scale);
#pragma omp parallel for schedule(static)
    for (int64_t a = 0; a < n; ++a) S[a] = overlap_one(c.A9, centers, c.norm, pi[a], pj[a]);
    chart_free(&c);
}

/* ---------------------------------------------------------------- screening */

int64_t orc_count_significant(int64_t M, const double* quat, const double* log_scale,
                              const double* centers, double eps, int unique) {
    Chart c = chart_alloc(M, quat, log_scale);
    int64_t tot = 0;
#pragma omp parallel for schedule(dynamic, 16) reduction(+ : tot)
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = unique ? i : 0; j < M; ++j)
            if (fabs(overlap_one(c.A9, centers, c.norm, (int)i, (int)j)) > eps) ++tot;
    chart_free(&c);
    return tot;
}

typedef struct { int64_t flat; double val; } FlatVal;

static int by_val_desc(const void* a, const void* b) {
    const FlatVal* x = (const FlatVal*)a;
    const FlatVal* y = (const FlatVal*)b;
    if (x->val > y->val) return -1;
    if (x->val < y->val) return 1;
    return (x->flat < y->flat) ? -1 : (x->flat > y->flat);   /* stable: original (flat) order */
}

static int by_flat(const void* a, const void* b) {
    int64_t x = *(const int64_t*)a, y = *(const int64_t*)b;
    return (x < y) ? -1 : (x > y);
}

/* gs_dft/screening/pairs.py:90-100,318-322 */
static void decode(const int64_t* flat, int64_t k, int64_t M, int64_t pad_to, int unique,
                   int32_t* pi, int32_t* pj, double* w) {
    for (int64_t a = 0; a < k; ++a) {
        pi[a] = (int32_t)(flat[a] / M);
        pj[a] = (int32_t)(flat[a] % M);
        w[a] = unique ? (pi[a] == pj[a] ? 1.0 : 2.0) : 1.0;
    }
    for (int64_t a = k; a < pad_to; ++a) { pi[a] = 0; pj[a] = 0; w[a] = 0.0; }
}

/* Per-row significant counts of the candidate space (pairs.py:103-118, one row at a time). */
static void row_counts(int64_t M, const Chart* c, const double* centers, double eps, int unique,
                       int64_t* cnt) {
#pragma omp parallel for schedule(dynamic, 8)
    for (int64_t i = 0; i < M; ++i) {
        int64_t k = 0;
        for (int64_t j = unique ? i : 0; j < M; ++j)
            if (fabs(overlap_one(c->A9, centers, c->norm, (int)i, (int)j)) > eps) ++k;
        cnt[i] = k;
    }
}

int orc_neighbor_pairs(int64_t M, const double* quat, const double* log_scale,
                       const double* centers, double eps, int64_t pad_to, int unique,
                       int32_t* pi, int32_t* pj, double* weight, int64_t* n_out, int64_t* n_sig) {
    int64_t n_all = unique ? M * (M + 1) / 2 : M * M;
    /* pairs.py:260-272: every pair significant and the pad covers them -> repeat/tile order */
    if (eps < 0.0 && (pad_to < 0 || pad_to >= n_all)) {
        int64_t a = 0;
        for (int64_t i = 0; i < M; ++i)
            for (int64_t j = unique ? i : 0; j < M; ++j, ++a) {
                pi[a] = (int32_t)i;
                pj[a] = (int32_t)j;
                weight[a] = unique ? (i == j ? 1.0 : 2.0) : 1.0;
            }
        int64_t len = pad_to < 0 ? n_all : pad_to;
        for (; a < len; ++a) { pi[a] = 0; pj[a] = 0; weight[a] = 0.0; }
        *n_out = len;
        *n_sig = n_all;
        return 0;
    }
    Chart c = chart_alloc(M, quat, log_scale);
    /* ascending flat i*M + j with their |S| (pairs.py:50-87 emits exactly this order): per-row
     * counts, their prefix sum, then every row fills its own segment in column order */
    int64_t* off = (int64_t*)malloc(sizeof(int64_t) * (size_t)(M + 1));
    row_counts(M, &c, centers, eps, unique, off + 1);
    off[0] = 0;
    for (int64_t i = 0; i < M; ++i) off[i + 1] += off[i];
    const int64_t cnt = off[M];
    FlatVal* sig = (FlatVal*)malloc(sizeof(FlatVal) * (size_t)(cnt > 0 ? cnt : 1));
#pragma omp parallel for schedule(dynamic, 8)
    for (int64_t i = 0; i < M; ++i) {
        int64_t a = off[i];
        for (int64_t j = unique ? i : 0; j < M; ++j) {
            double s = fabs(overlap_one(c.A9, centers, c.norm, (int)i, (int)j));
            if (s > eps) {
                sig[a].flat = i * M + j;
                sig[a].val = s;
                ++a;
            }
        }
    }
    free(off);
    chart_free(&c);
    *n_sig = cnt;
    if (pad_to < 0) pad_to = cnt;                         /* pairs.py:278-282 */
    *n_out = pad_to;
    int64_t* flat = (int64_t*)malloc(sizeof(int64_t) * (cnt > 0 ? cnt : 1));
    int rc = 0;
    if (cnt > pad_to) {
        /* pairs.py:155-164: raise beyond 2x the pad, else keep the pad_to largest |S| and
         * re-sort them by flat index */
        if (cnt > 2 * pad_to) {
            rc = 2;
        } else {
            qsort(sig, (size_t)cnt, sizeof(FlatVal), by_val_desc);
            for (int64_t a = 0; a < pad_to; ++a) flat[a] = sig[a].flat;
            qsort(flat, (size_t)pad_to, sizeof(int64_t), by_flat);
            decode(flat, pad_to, M, pad_to, unique, pi, pj, weight);
        }
    } else {
        for (int64_t a = 0; a < cnt; ++a) flat[a] = sig[a].flat;
        decode(flat, cnt, M, pad_to, unique, pi, pj, weight);
    }
    free(flat);
    free(sig);
    return rc;
}

/* Knife-edge audit of the threshold: over every candidate (j >= i when unique), the number with
 * ||S| - eps| <= rel_tol * eps and the smallest ||S| - eps| / eps. */
void orc_screen_margin(int64_t M, const double* quat, const double* log_scale,
                       const double* centers, double eps, int unique, double rel_tol,
                       int64_t* n_close, double* min_gap) {
    Chart c = chart_alloc(M, quat, log_scale);
    int64_t close = 0;
    double gap = INFINITY;
#pragma omp parallel for schedule(dynamic, 8) reduction(+ : close) reduction(min : gap)
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = unique ? i : 0; j < M; ++j) {
            double r = fabs(fabs(overlap_one(c.A9, centers, c.norm, (int)i, (int)j)) - eps) / eps;
            if (r <= rel_tol) ++close;
            if (r < gap) gap = r;
        }
    chart_free(&c);
    *n_close = close;
    *min_gap = gap;
}

/* The spatial candidate rules against the significant set, by brute force over the candidate
 * space (j >= i when unique), with L = max(-ln eps, 1e-12) and lmin_i = exp(min_k l_ik):
 *   reference rule (pairs.py:167-197, grid.py:76-82): |mu_i - mu_j| < safety (rc_i + rc_j),
 *     rc_i = sqrt(L / lmin_i);
 *   bound rule: |mu_i - mu_j|^2 < L (1/lmin_i + 1/lmin_j).
 * Outputs: significant pairs, candidates of each rule, significant pairs each rule misses, and
 * the largest |d|^2 / (L (1/lmin_i + 1/lmin_j)) over the significant pairs. */
void orc_spatial_audit(int64_t M, const double* quat, const double* log_scale,
                       const double* centers, double eps, int unique, double safety,
                       int64_t* n_sig, int64_t* n_cand_ref, int64_t* n_miss_ref,
                       int64_t* n_cand_bound, int64_t* n_miss_bound, double* max_ratio) {
    Chart c = chart_alloc(M, quat, log_scale);
    const double L = fmax(-log(eps), 1e-12);
    double* inv = (double*)malloc(sizeof(double) * (size_t)(M > 0 ? M : 1));
    for (int64_t m = 0; m < M; ++m) {
        const double* l = log_scale + 3 * m;
        inv[m] = 1.0 / exp(fmin(l[0], fmin(l[1], l[2])));
    }
    int64_t ns = 0, cr = 0, mr = 0, cb = 0, mb = 0;
    double mx = 0.0;
#pragma omp parallel for schedule(dynamic, 8) reduction(+ : ns, cr, mr, cb, mb) reduction(max : mx)
    for (int64_t i = 0; i < M; ++i)
        for (int64_t j = unique ? i : 0; j < M; ++j) {
            const double* a = centers + 3 * i;
            const double* b = centers + 3 * j;
            const double d2 = (a[0] - b[0]) * (a[0] - b[0]) + (a[1] - b[1]) * (a[1] - b[1])
                            + (a[2] - b[2]) * (a[2] - b[2]);
            const int ref = sqrt(d2) < safety * (sqrt(L * inv[i]) + sqrt(L * inv[j]));
            const double ratio = d2 / (L * (inv[i] + inv[j]));
            const int bnd = ratio < 1.0;
            const int sig = fabs(overlap_one(c.A9, centers, c.norm, (int)i, (int)j)) > eps;
            cr += ref;
            cb += bnd;
            if (sig) {
                ++ns;
                mr += !ref;
                mb += !bnd;
                if (ratio > mx) mx = ratio;
            }
        }
    free(inv);
    chart_free(&c);
    *n_sig = ns;
    *n_cand_ref = cr;
    *n_miss_ref = mr;
    *n_cand_bound = cb;
    *n_miss_bound = mb;
    *max_ratio = mx;
}

/* ---------------------------------------------------------------- product aux */

/* gs_dft/basis/isotropic.py:81-116 with diagonal_only (pi = pj = arange(M)): alpha_0 =
 * det3(A_i + A_i)^(1/3) at the product centre of the self-pair. */
void orc_product_aux(int64_t M, const double* quat, const double* log_scale,
                     const double* centers, const double* scales, int n_scales,
                     double* log_alpha, double* aux_centers) {
    Chart c = chart_alloc(M, quat, log_scale);
    for (int64_t m = 0; m < M; ++m) {
        double Ah[9], Pc[3], KN;
        const double* A = c.A9 + 9 * m;
        pair_q(A, A, centers + 3 * m, centers + 3 * m, c.norm[m], c.norm[m], Ah, Pc, &KN, NULL);
        double alpha0 = pow(det3(Ah), 1.0 / 3.0);
        for (int s = 0; s < n_scales; ++s) {
            int64_t o = (int64_t)s * M + m;
            log_alpha[o] = log(alpha0 * scales[s]);
            aux_centers[3 * o] = Pc[0];
            aux_centers[3 * o + 1] = Pc[1];
            aux_centers[3 * o + 2] = Pc[2];
        }
    }
    chart_free(&c);
}

/* gs_dft/basis/isotropic.py:106-116 with diagonal_only=False and a pair list: one aux per listed
 * pair a at its product centre with alpha_0 = det3(A_i + A_j)^(1/3), alpha_0 = 1 where valid[a]
 * is 0 (valid may be NULL: every entry live), scale-major over the n_scales scales. */
void orc_product_aux_pairs(int64_t M, const double* quat, const double* log_scale,
                           const double* centers, int64_t n, const int32_t* pi,
                           const int32_t* pj, const double* valid, const double* scales,
                           int n_scales, double* log_alpha, double* aux_centers) {
    Chart c = chart_alloc(M, quat, log_scale);
    for (int64_t a = 0; a < n; ++a) {
        const int i = pi[a], j = pj[a];
        double Ah[9], Pc[3], KN;
        pair_q(c.A9 + 9 * i, c.A9 + 9 * j, centers + 3 * i, centers + 3 * j, c.norm[i],
               c.norm[j], Ah, Pc, &KN, NULL);
        double alpha0 = pow(det3(Ah), 1.0 / 3.0);
        if (valid && valid[a] == 0.0) alpha0 = 1.0;
        for (int s = 0; s < n_scales; ++s) {
            int64_t o = (int64_t)s * n + a;
            log_alpha[o] = log(alpha0 * scales[s]);
            aux_centers[3 * o] = Pc[0];
            aux_centers[3 * o + 1] = Pc[1];
            aux_centers[3 * o + 2] = Pc[2];
        }
    }
    chart_free(&c);
}

/* ---------------------------------------------------------------- metric */

/* Boys F0 = 0.5 sqrt(pi/T) erf(sqrt(T)); the reference calls dftax.energy.boys.boys(0, T)
 * (gs_dft/coulomb/ri.py:74), which is not available here. */
double orc_boys0(double T) {
    if (T < 1e-12) return 1.0 - T / 3.0;
    double x = sqrt(T);
    return 0.5 * sqrt(M_PI / T) * erf(x);
}

/* gs_dft/coulomb/ri.py:63-76 (omega=None) for one (row, col) element. */
/* gs_dft/coulomb/ri.py:63-76: 1/r for omega = 0; erf(omega r)/r otherwise (ri.py:70-72:
 * z = omega^2 / (omega^2 + rho), F0 = sqrt(z) boys0(z T)). */
static double metric_one(double g1, const double* P1, double KN1, double g2, const double* P2,
                         double KN2, double omega) {
    double gab = g1 * g2;
    double gsum = g1 + g2;
    double dx = P1[0] - P2[0], dy = P1[1] - P2[1], dz = P1[2] - P2[2];
    double PQ2 = dx * dx + dy * dy + dz * dz;
    double rho = gab / gsum;
    double T = rho * PQ2;
    double F0;
    if (omega != 0.0) {
        double z = (omega * omega) / (omega * omega + rho);
        F0 = sqrt(z) * orc_boys0(z * T);
    } else {
        F0 = orc_boys0(T);
    }
    double coul = (2.0 * pow(M_PI, 2.5)) / (gab * sqrt(gsum)) * F0;
    return (KN1 * KN2) * coul;
}

void orc_aux_metric(int64_t N, const double* log_alpha, const double* centers, double lam,
                    double omega, double* V) {
    double* beta = (double*)malloc(sizeof(double) * (N > 0 ? N : 1));
    double* KN = (double*)malloc(sizeof(double) * (N > 0 ? N : 1));
    for (int64_t p = 0; p < N; ++p) {          /* gs_dft/basis/isotropic.py:30-39 */
        beta[p] = exp(log_alpha[p]);
        KN[p] = pow(2.0 * beta[p] / M_PI, 0.75);
    }
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < N; ++p)
        for (int64_t q = 0; q < N; ++q)
            V[p * N + q] = metric_one(beta[p], centers + 3 * p, KN[p], beta[q], centers + 3 * q,
                                      KN[q], omega);
    if (lam != 0.0)
        for (int64_t p = 0; p < N; ++p) V[p * N + p] += lam;   /* ri.py:243-250 */
    free(beta);
    free(KN);
}

/* Rows rows[0..nrows) of the same metric: V (nrows, N), lam added where the row meets the
 * diagonal. */
void orc_aux_metric_rows(int64_t N, const double* log_alpha, const double* centers, double lam,
                         double omega, int64_t nrows, const int64_t* rows, double* V) {
    double* beta = (double*)malloc(sizeof(double) * (N > 0 ? N : 1));
    double* KN = (double*)malloc(sizeof(double) * (N > 0 ? N : 1));
    for (int64_t p = 0; p < N; ++p) {          /* gs_dft/basis/isotropic.py:30-39 */
        beta[p] = exp(log_alpha[p]);
        KN[p] = pow(2.0 * beta[p] / M_PI, 0.75);
    }
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < nrows; ++r) {
        const int64_t p = rows[r];
        for (int64_t q = 0; q < N; ++q)
            V[r * N + q] = metric_one(beta[p], centers + 3 * p, KN[p], beta[q], centers + 3 * q,
                                      KN[q], omega);
        if (lam != 0.0) V[r * N + p] += lam;   /* ri.py:243-250 */
    }
    free(beta);
    free(KN);
}

/* ---------------------------------------------------------------- Cholesky + solve */

int orc_cholesky(int64_t N, double* V) {
    /* Left-looking row-oriented Cholesky-Banachiewicz; row-major lower. */
    for (int64_t i = 0; i < N; ++i) {
        double* Li = V + i * N;
        for (int64_t j = 0; j <= i; ++j) {
            const double* Lj = V + j * N;
            double s = Li[j];
            for (int64_t k = 0; k < j; ++k) s -= Li[k] * Lj[k];
            if (i == j) {
                if (!(s > 0.0)) return 1;
                Li[i] = sqrt(s);
            } else {
                Li[j] = s / Lj[j];
            }
        }
    }
    for (int64_t i = 0; i < N; ++i)
        for (int64_t j = i + 1; j < N; ++j) V[i * N + j] = 0.0;
    return 0;
}

void orc_cho_solve(int64_t N, const double* L, const double* gamma, double* d) {
    double* y = (double*)malloc(sizeof(double) * (N > 0 ? N : 1));
    for (int64_t i = 0; i < N; ++i) {                 /* L y = gamma */
        double s = gamma[i];
        for (int64_t k = 0; k < i; ++k) s -= L[i * N + k] * y[k];
        y[i] = s / L[i * N + i];
    }
    for (int64_t i = N - 1; i >= 0; --i) {            /* L^T d = y */
        double s = y[i];
        for (int64_t k = i + 1; k < N; ++k) s -= L[k * N + i] * d[k];
        d[i] = s / L[i * N + i];
    }
    free(y);
}

/* ---------------------------------------------------------------- three-centre */

typedef struct {
    double A[9];          /* product precision */
    double P[3];          /* product centre */
    double KN;            /* N_i N_j K */
    double I1, I2, I3;    /* rotation invariants of A */
} PairRec;

static void pair_rec(const double* A9, const double* mu, const double* norm, int i, int j,
                     PairRec* r) {
    pair_q(A9 + 9 * i, A9 + 9 * j, mu + 3 * i, mu + 3 * j, norm[i], norm[j], r->A, r->P, &r->KN,
           NULL);
    const double* A = r->A;
    r->I1 = A[0] + A[4] + A[8];
    r->I2 = A[0] * A[4] + A[0] * A[8] + A[4] * A[8] - A[1] * A[3] - A[2] * A[6] - A[5] * A[7];
    r->I3 = det3(A);
}

/* ri.py:150 pref = 2 pi^3 / sqrt(pi) */
static double pref3c(void) { return 2.0 * (M_PI * M_PI * M_PI) / sqrt(M_PI); }

/* The node sum of gs_dft/coulomb/ri.py:172-184 for one (aux, pair) in invariant form. */
static double node_sum(const double* tq, const double* wq, double beta, const double* R,
                       const PairRec* r) {
    double d[3] = {R[0] - r->P[0], R[1] - r->P[1], R[2] - r->P[2]};
    double Ad[3];
    matvec3(r->A, d, Ad);
    double q0 = d[0] * d[0] + d[1] * d[1] + d[2] * d[2];
    double q1 = d[0] * Ad[0] + d[1] * Ad[1] + d[2] * Ad[2];
    double q2 = Ad[0] * Ad[0] + Ad[1] * Ad[1] + Ad[2] * Ad[2];
    double F = 0.0;
    for (int t = 0; t < NQ; ++t) {
        double t2 = tq[t] * tq[t];
        double a = beta + t2, c = t2 * beta;
        double a2 = a * a, c2 = c * c;
        double D = a2 * a * r->I3 + a2 * c * r->I2 + a * c2 * r->I1 + c2 * c;
        double Nn = beta * (a2 * r->I3 * q0 + a * c * (r->I1 * q1 - q2) + c2 * q1);
        F += wq[t] * sqrt(1.0 / D) * exp(-t2 * Nn / D);
    }
    return F;
}

typedef struct {
    int64_t N;
    double* beta;
    double* KN;
} AuxQ;

static AuxQ aux_alloc(int64_t N, const double* log_alpha) {
    AuxQ q;
    q.N = N;
    q.beta = (double*)malloc(sizeof(double) * (N > 0 ? N : 1));
    q.KN = (double*)malloc(sizeof(double) * (N > 0 ? N : 1));
    for (int64_t p = 0; p < N; ++p) {
        q.beta[p] = exp(log_alpha[p]);
        q.KN[p] = pow(2.0 * q.beta[p] / M_PI, 0.75);
    }
    return q;
}

static void aux_free(AuxQ* q) { free(q->beta); free(q->KN); }

void orc_three_center_block(int64_t M, const double* quat, const double* log_scale,
                            const double* centers, int64_t N, const double* log_alpha,
                            const double* aux_centers, int64_t n, const int32_t* pi,
                            const int32_t* pj, double* block) {
    double tq[NQ], wq[NQ];
    node_table(tq, wq);
    Chart c = chart_alloc(M, quat, log_scale);
    AuxQ aq = aux_alloc(N, log_alpha);
    PairRec* pr = (PairRec*)malloc(sizeof(PairRec) * (n > 0 ? n : 1));
    for (int64_t a = 0; a < n; ++a) pair_rec(c.A9, centers, c.norm, pi[a], pj[a], pr + a);
    double pref = pref3c();
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < N; ++p)
        for (int64_t a = 0; a < n; ++a)
            block[p * n + a] = (aq.KN[p] * pr[a].KN) * pref
                             * node_sum(tq, wq, aq.beta[p], aux_centers + 3 * p, pr + a);
    free(pr);
    aux_free(&aq);
    chart_free(&c);
}

/* ri.py:456: q_a = w_a sum_o occ_o C_io C_jo */
static double pair_density(int64_t k, const double* C, const double* occ, int i, int j) {
    double s = 0.0;
    for (int64_t o = 0; o < k; ++o) s += occ[o] * C[i * k + o] * C[j * k + o];
    return s;
}

void orc_gamma(int64_t M, const double* quat, const double* log_scale, const double* centers,
               int64_t k, const double* C, const double* occ, int64_t N,
               const double* log_alpha, const double* aux_centers, int64_t n,
               const int32_t* pi, const int32_t* pj, const double* weight, double* gamma) {
    double tq[NQ], wq[NQ];
    node_table(tq, wq);
    Chart c = chart_alloc(M, quat, log_scale);
    AuxQ aq = aux_alloc(N, log_alpha);
    PairRec* pr = (PairRec*)malloc(sizeof(PairRec) * (n > 0 ? n : 1));
    double* qa = (double*)malloc(sizeof(double) * (n > 0 ? n : 1));
#pragma omp parallel for schedule(static)
    for (int64_t a = 0; a < n; ++a) {
        pair_rec(c.A9, centers, c.norm, pi[a], pj[a], pr + a);
        qa[a] = weight[a] * pair_density(k, C, occ, pi[a], pj[a]);
    }
    double pref = pref3c();
    /* Pair blocks that stay in cache while every aux row sweeps them; each gamma_P still sums its
     * pairs in list order. */
    const int64_t kBlk = 2048;
    for (int64_t p = 0; p < N; ++p) gamma[p] = 0.0;
    for (int64_t a0 = 0; a0 < n; a0 += kBlk) {
        const int64_t a1 = a0 + kBlk < n ? a0 + kBlk : n;
#pragma omp parallel for schedule(static)
        for (int64_t p = 0; p < N; ++p) {
            double g = gamma[p];
            for (int64_t a = a0; a < a1; ++a) {
                if (qa[a] == 0.0) continue;      /* zero-weight (padding) pairs add exactly 0 */
                double blk = (aq.KN[p] * pr[a].KN) * pref
                           * node_sum(tq, wq, aq.beta[p], aux_centers + 3 * p, pr + a);
                g += blk * qa[a];
            }
            gamma[p] = g;
        }
    }
    free(qa);
    free(pr);
    aux_free(&aq);
    chart_free(&c);
}

/* ---------------------------------------------------------------- reverse mode */

/* Gradient matrices are symmetric and enter as dE = sum_kl G_kl dA_kl over all nine entries. */
static void add_sym_outer(double* G, double s, const double* x, const double* y) {
    for (int k = 0; k < 3; ++k)
        for (int l = 0; l < 3; ++l) G[3 * k + l] += 0.5 * s * (x[k] * y[l] + y[k] * x[l]);
}

/* Per (aux, pair): accumulate the derivative of F = node sum w.r.t. I1, I2, I3, q0, q1, q2. */
static double node_sum_grad(const double* tq, const double* wq, double beta, double q0, double q1,
                            double q2, const PairRec* r, double* gI, double* gq) {
    double F = 0.0;
    gI[0] = gI[1] = gI[2] = 0.0;
    gq[0] = gq[1] = gq[2] = 0.0;
    for (int t = 0; t < NQ; ++t) {
        double t2 = tq[t] * tq[t];
        double a = beta + t2, c = t2 * beta;
        double a2 = a * a, c2 = c * c;
        double D = a2 * a * r->I3 + a2 * c * r->I2 + a * c2 * r->I1 + c2 * c;
        double Nn = beta * (a2 * r->I3 * q0 + a * c * (r->I1 * q1 - q2) + c2 * q1);
        double f = wq[t] * sqrt(1.0 / D) * exp(-t2 * Nn / D);
        F += f;
        double fD = f * (-0.5 / D + t2 * Nn / (D * D));       /* df/dD  */
        double fN = -f * t2 / D;                              /* df/dNn */
        gI[0] += fD * a * c2 + fN * beta * a * c * q1;        /* d/dI1 */
        gI[1] += fD * a2 * c;                                 /* d/dI2 */
        gI[2] += fD * a2 * a + fN * beta * a2 * q0;           /* d/dI3 */
        gq[0] += fN * beta * a2 * r->I3;                      /* d/dq0 */
        gq[1] += fN * beta * (a * c * r->I1 + c2);            /* d/dq1 */
        gq[2] += -fN * beta * a * c;                          /* d/dq2 */
    }
    return F;
}

void orc_gamma_vjp(int64_t M, const double* quat, const double* log_scale, const double* centers,
                   int64_t k, const double* C, const double* occ, int64_t N,
                   const double* log_alpha, const double* aux_centers, int64_t n,
                   const int32_t* pi, const int32_t* pj, const double* weight,
                   const double* dgamma, double* J, double* dquat, double* dlog_scale,
                   double* dcenters, double* dC) {
    double tq[NQ], wq[NQ];
    node_table(tq, wq);
    Chart c = chart_alloc(M, quat, log_scale);
    AuxQ aq = aux_alloc(N, log_alpha);
    double pref = pref3c();
    /* per-splat accumulators: G_A (9), g_mu (3), g_N (1) */
    double* GA = (double*)calloc((size_t)(9 * M + 1), sizeof(double));
    double* gmu = (double*)calloc((size_t)(3 * M + 1), sizeof(double));
    double* gN = (double*)calloc((size_t)(M + 1), sizeof(double));
    /* per-pair outputs of the parallel phase */
    double* pairG = (double*)calloc((size_t)(n > 0 ? n : 1) * 26, sizeof(double));

#pragma omp parallel for schedule(dynamic, 4)
    for (int64_t a = 0; a < n; ++a) {
        int i = pi[a], j = pj[a];
        double* out = pairG + 26 * a;
        if (weight[a] == 0.0) {             /* padding: no contribution, J defined as 0 */
            J[a] = 0.0;
            continue;
        }
        double qd = pair_density(k, C, occ, i, j);
        double qa = weight[a] * qd;
        PairRec r;
        pair_rec(c.A9, centers, c.norm, i, j, &r);
        double jt = 0.0;                    /* sum_P dgamma_P KN_P F */
        double GAh[9] = {0}, gP[3] = {0}, gI[3] = {0};
        for (int64_t p = 0; p < N; ++p) {
            const double* R = aux_centers + 3 * p;
            double d[3] = {R[0] - r.P[0], R[1] - r.P[1], R[2] - r.P[2]};
            double Ad[3], AAd[3];
            matvec3(r.A, d, Ad);
            matvec3(r.A, Ad, AAd);
            double q0 = d[0] * d[0] + d[1] * d[1] + d[2] * d[2];
            double q1 = d[0] * Ad[0] + d[1] * Ad[1] + d[2] * Ad[2];
            double q2 = Ad[0] * Ad[0] + Ad[1] * Ad[1] + Ad[2] * Ad[2];
            double lgI[3], lgq[3];
            double F = node_sum_grad(tq, wq, aq.beta[p], q0, q1, q2, &r, lgI, lgq);
            double u = dgamma[p] * aq.KN[p];
            jt += u * F;
            double s = u;                           /* times q_a KN_a pref, applied below */
            for (int m = 0; m < 3; ++m) gI[m] += s * lgI[m];
            /* q0 = |d|^2, q1 = d.A d, q2 = |A d|^2 with d = R - P */
            for (int m = 0; m < 3; ++m)
                gP[m] += s * (-2.0 * lgq[0] * d[m] - 2.0 * lgq[1] * Ad[m] - 2.0 * lgq[2] * AAd[m]);
            add_sym_outer(GAh, s * lgq[1], d, d);
            add_sym_outer(GAh, s * lgq[2], Ad, d);
            add_sym_outer(GAh, s * lgq[2], d, Ad);
        }
        double scale = qa * r.KN * pref;
        J[a] = r.KN * pref * jt;
        double gKN = qa * pref * jt;
        /* invariants -> A: dI1 = I, dI2 = I1 I - A, dI3 = adj(A) */
        double adj[9];
        adj3(r.A, adj);
        for (int m = 0; m < 9; ++m) {
            double eye = (m == 0 || m == 4 || m == 8) ? 1.0 : 0.0;
            GAh[m] = scale * (GAh[m] + gI[0] * eye + gI[1] * (r.I1 * eye - r.A[m]) + gI[2] * adj[m]);
        }
        for (int m = 0; m < 3; ++m) gP[m] *= scale;
        memcpy(out, GAh, 9 * sizeof(double));
        memcpy(out + 9, gP, 3 * sizeof(double));
        out[12] = gKN;
    }

    /* pair-quantity VJP (stream.py:203-215) and deterministic per-splat sums in pair order */
    for (int64_t a = 0; a < n; ++a) {
        if (weight[a] == 0.0) continue;
        int i = pi[a], j = pj[a];
        const double* in = pairG + 26 * a;
        const double *Ai = c.A9 + 9 * i, *Aj = c.A9 + 9 * j;
        const double *mui = centers + 3 * i, *muj = centers + 3 * j;
        double Gh[9], gPc[3], gKN = in[12];
        memcpy(Gh, in, sizeof Gh);
        memcpy(gPc, in + 9, sizeof gPc);
        double Ah[9], Pc[3], KN;
        pair_q(Ai, Aj, mui, muj, c.norm[i], c.norm[j], Ah, Pc, &KN, NULL);
        double Gi[9] = {0}, Gj[9] = {0};
        double gmi[3] = {0}, gmj[3] = {0};
        /* KN = N_i N_j K, K = exp(-e) */
        double d[3] = {mui[0] - muj[0], mui[1] - muj[1], mui[2] - muj[2]};
        double Ajd[3], Aid[3], u[3], v[3], Aiu[3], Ajv[3];
        matvec3(Aj, d, Ajd);
        matvec3(Ai, d, Aid);
        solve3(Ah, Ajd, u);
        solve3(Ah, Aid, v);
        matvec3(Ai, u, Aiu);
        matvec3(Aj, v, Ajv);
        double e = d[0] * Aiu[0] + d[1] * Aiu[1] + d[2] * Aiu[2];
        double K = exp(-e);
        gN[i] += gKN * c.norm[j] * K;
        gN[j] += gKN * c.norm[i] * K;
        double ge = -gKN * KN;
        for (int m = 0; m < 3; ++m) {
            double gd = ge * (Aiu[m] + Ajv[m]);
            gmi[m] += gd;
            gmj[m] -= gd;
        }
        add_sym_outer(Gi, ge, d, u);
        add_sym_outer(Gj, ge, v, d);
        double Gv[9] = {0};
        add_sym_outer(Gv, -ge, v, u);
        for (int m = 0; m < 9; ++m) Gh[m] += Gv[m];
        /* P = Ah^-1 (Ai mu_i + Aj mu_j) */
        double y[3];
        solve3(Ah, gPc, y);
        add_sym_outer(Gh, -1.0, y, Pc);
        add_sym_outer(Gi, 1.0, y, mui);
        add_sym_outer(Gj, 1.0, y, muj);
        double Aiy[3], Ajy[3];
        matvec3(Ai, y, Aiy);
        matvec3(Aj, y, Ajy);
        for (int m = 0; m < 3; ++m) { gmi[m] += Aiy[m]; gmj[m] += Ajy[m]; }
        /* Ah = Ai + Aj */
        for (int m = 0; m < 9; ++m) { Gi[m] += Gh[m]; Gj[m] += Gh[m]; }
        for (int m = 0; m < 9; ++m) { GA[9 * i + m] += Gi[m]; GA[9 * j + m] += Gj[m]; }
        for (int m = 0; m < 3; ++m) { gmu[3 * i + m] += gmi[m]; gmu[3 * j + m] += gmj[m]; }
    }

    /* chart VJP (spectral.py:33-40,72-82) */
    for (int64_t m = 0; m < M; ++m) {
        const double* q = quat + 4 * m;
        const double* l = log_scale + 3 * m;
        double R[9], qn[4], nrm;
        quat_rotation(q, R, qn, &nrm);
        double a[3] = {exp(l[0]), exp(l[1]), exp(l[2])};
        const double* G = GA + 9 * m;
        double GR[9];
        for (int r = 0; r < 3; ++r)
            for (int cc = 0; cc < 3; ++cc)
                GR[3 * r + cc] = G[3 * r] * R[cc] + G[3 * r + 1] * R[3 + cc] + G[3 * r + 2] * R[6 + cc];
        double Nm = c.norm[m];
        for (int jx = 0; jx < 3; ++jx) {
            double ga = R[jx] * GR[jx] + R[3 + jx] * GR[3 + jx] + R[6 + jx] * GR[6 + jx];
            dlog_scale[3 * m + jx] = a[jx] * ga + gN[m] * Nm * 0.25;
        }
        double gR[9];
        for (int r = 0; r < 3; ++r)
            for (int cc = 0; cc < 3; ++cc) gR[3 * r + cc] = 2.0 * a[cc] * GR[3 * r + cc];
        double w = qn[0], x = qn[1], yq = qn[2], z = qn[3];
        double gw = 2 * (-z * gR[1] + yq * gR[2] + z * gR[3] - x * gR[5] - yq * gR[6] + x * gR[7]);
        double gx = 2 * (yq * gR[1] + z * gR[2] + yq * gR[3] - 2 * x * gR[4] - w * gR[5]
                         + z * gR[6] + w * gR[7] - 2 * x * gR[8]);
        double gy = 2 * (-2 * yq * gR[0] + x * gR[1] + w * gR[2] + x * gR[3] + z * gR[5]
                         - w * gR[6] + z * gR[7] - 2 * yq * gR[8]);
        double gz = 2 * (-2 * z * gR[0] - w * gR[1] + x * gR[2] + w * gR[3] - 2 * z * gR[4]
                         + yq * gR[5] + x * gR[6] + yq * gR[7]);
        double gqn[4] = {gw, gx, gy, gz};
        double den = nrm + 1e-12;
        double dot = q[0] * gqn[0] + q[1] * gqn[1] + q[2] * gqn[2] + q[3] * gqn[3];
        for (int t = 0; t < 4; ++t)
            dquat[4 * m + t] = gqn[t] / den - q[t] * dot / (nrm * den * den);
        for (int t = 0; t < 3; ++t) dcenters[3 * m + t] = gmu[3 * m + t];
    }

    /* dC (ri.py:456): dE/dC_ko = occ_o sum_a J_a w_a (d_{k,i_a} C_{j_a o} + d_{k,j_a} C_{i_a o}) */
    memset(dC, 0, sizeof(double) * (size_t)(M * k));
    for (int64_t a = 0; a < n; ++a) {
        int i = pi[a], j = pj[a];
        double s = J[a] * weight[a];
        if (s == 0.0) continue;
        for (int64_t o = 0; o < k; ++o) {
            dC[i * k + o] += s * occ[o] * C[j * k + o];
            dC[j * k + o] += s * occ[o] * C[i * k + o];
        }
    }
    free(pairG);
    free(GA);
    free(gmu);
    free(gN);
    aux_free(&aq);
    chart_free(&c);
}

/* ---------------------------------------------------------------- nuclear attraction */

/* gs_dft/screening/pairs.py:348-370 in its own (literal) form: per node B = A_ij + t^2 I,
 * invdet = 1/det(B), qf = d.adj(B).d, expo = t^2 |d|^2 - t^4 qf invdet, and
 * vA = (2/sqrt(pi)) sum_t w_t pi^1.5 sqrt(invdet) exp(-expo); V = -sum_A Z_A vA N_i N_j K. */
static double nuclear_one(const double* tq, const double* wq, const double* A, const double* P,
                          double NK, int64_t n_atoms, const double* coords,
                          const double* charges) {
    double V = 0.0;
    for (int64_t at = 0; at < n_atoms; ++at) {
        const double* R = coords + 3 * at;
        double d[3] = {P[0] - R[0], P[1] - R[1], P[2] - R[2]};
        double d2 = d[0] * d[0] + d[1] * d[1] + d[2] * d[2];
        double vA = 0.0;
        for (int t = 0; t < NQ; ++t) {
            double t2 = tq[t] * tq[t];
            double B[9];
            memcpy(B, A, sizeof B);
            B[0] += t2; B[4] += t2; B[8] += t2;
            double invdet = 1.0 / det3(B);
            double adj[9], ad[3];
            adj3(B, adj);
            matvec3(adj, d, ad);
            double qf = d[0] * ad[0] + d[1] * ad[1] + d[2] * ad[2];
            double expo = t2 * d2 - (t2 * t2) * qf * invdet;
            vA += (wq[t] * PI15) * sqrt(invdet) * exp(-expo);
        }
        vA *= 2.0 / sqrt(M_PI);
        V += charges[at] * vA;
    }
    return -V * NK;
}

void orc_nuclear_pairs(int64_t M, const double* quat, const double* log_scale,
                       const double* centers, int64_t n, const int32_t* pi, const int32_t* pj,
                       int64_t n_atoms, const double* coords, const double* charges, double* V) {
    double tq[NQ], wq[NQ];
    node_table(tq, wq);
    Chart c = chart_alloc(M, quat, log_scale);
#pragma omp parallel for schedule(static)
    for (int64_t a = 0; a < n; ++a) {
        double Ah[9], P[3], KN;
        pair_q(c.A9 + 9 * pi[a], c.A9 + 9 * pj[a], centers + 3 * pi[a], centers + 3 * pj[a],
               c.norm[pi[a]], c.norm[pj[a]], Ah, P, &KN, NULL);
        V[a] = nuclear_one(tq, wq, Ah, P, KN, n_atoms, coords, charges);
    }
    chart_free(&c);
}

/* gs_dft/screening/pairs.py:409-440: E = sum_a w_a P_a V_a, P_a = sum_o occ_o C_io C_jo. */
double orc_external_energy(int64_t M, const double* quat, const double* log_scale,
                           const double* centers, int64_t k, const double* C, const double* occ,
                           int64_t n, const int32_t* pi, const int32_t* pj, const double* weight,
                           int64_t n_atoms, const double* coords, const double* charges) {
    double* V = (double*)malloc(sizeof(double) * (n > 0 ? n : 1));
    orc_nuclear_pairs(M, quat, log_scale, centers, n, pi, pj, n_atoms, coords, charges, V);
    double E = 0.0;
    for (int64_t a = 0; a < n; ++a) {
        if (weight[a] == 0.0) continue;
        E += weight[a] * pair_density(k, C, occ, pi[a], pj[a]) * V[a];
    }
    free(V);
    return E;
}

/* ---------------------------------------------------------------- exact pair-pair Coulomb */

static void inv3m(const double* A, double* Ai) {
    double c[9];
    adj3(A, c);
    double det = det3(A);
    for (int m = 0; m < 9; ++m) Ai[m] = c[m] / det;
}

/* (a|b) of gs_dft/coulomb/stream.py:249-281 (full_eri_block_schur) for one pair-pair, node by
 * node in the Schur-complement form: X = A_a + t^2 I, u = X^-1 v_a, S = Y - t^4 X^-1 with
 * Y = A_b + t^2 I, w = t^2 u + v_b, quad = c.v - (v_a.u + w.S^-1 w), det G = det X det S. */
static double eri_schur_one(const double* tq, const double* wq, const PairRec* a,
                            const PairRec* b) {
    double va[3], vb[3];
    matvec3(a->A, a->P, va);
    matvec3(b->A, b->P, vb);
    double cv = (a->P[0] * va[0] + a->P[1] * va[1] + a->P[2] * va[2])
              + (b->P[0] * vb[0] + b->P[1] * vb[1] + b->P[2] * vb[2]);
    double coul = 0.0;
    for (int t = 0; t < NQ; ++t) {
        double t2 = tq[t] * tq[t];
        double X[9], Xi[9], u[3], Y[9], S[9], w[3], z[3];
        memcpy(X, a->A, sizeof X);
        X[0] += t2; X[4] += t2; X[8] += t2;
        inv3m(X, Xi);
        matvec3(Xi, va, u);
        double vau = va[0] * u[0] + va[1] * u[1] + va[2] * u[2];
        memcpy(Y, b->A, sizeof Y);
        Y[0] += t2; Y[4] += t2; Y[8] += t2;
        for (int m = 0; m < 9; ++m) S[m] = Y[m] - t2 * t2 * Xi[m];
        for (int m = 0; m < 3; ++m) w[m] = t2 * u[m] + vb[m];
        solve3(S, w, z);
        double quad = cv - (vau + (w[0] * z[0] + w[1] * z[1] + w[2] * z[2]));
        double detG = det3(X) * det3(S);
        double It = (M_PI * M_PI * M_PI) / sqrt(detG) * exp(-quad);
        coul += wq[t] * (2.0 / sqrt(M_PI)) * It;
    }
    return a->KN * b->KN * coul;
}

void orc_eri_block(int64_t M, const double* quat, const double* log_scale, const double* centers,
                   int64_t na, const int32_t* ai, const int32_t* aj, int64_t nb,
                   const int32_t* bi, const int32_t* bj, double* out) {
    double tq[NQ], wq[NQ];
    node_table(tq, wq);
    Chart c = chart_alloc(M, quat, log_scale);
    PairRec* ra = (PairRec*)malloc(sizeof(PairRec) * (na > 0 ? na : 1));
    PairRec* rb = (PairRec*)malloc(sizeof(PairRec) * (nb > 0 ? nb : 1));
    for (int64_t x = 0; x < na; ++x) pair_rec(c.A9, centers, c.norm, ai[x], aj[x], ra + x);
    for (int64_t x = 0; x < nb; ++x) pair_rec(c.A9, centers, c.norm, bi[x], bj[x], rb + x);
#pragma omp parallel for schedule(static)
    for (int64_t x = 0; x < na; ++x)
        for (int64_t y = 0; y < nb; ++y) out[x * nb + y] = eri_schur_one(tq, wq, ra + x, rb + y);
    free(ra);
    free(rb);
    chart_free(&c);
}

/* Jvec_a = sum_b (a|b) Pw_b with Pw_b = w_b sum_o occ_o C_io C_jo (stream.py:296-320), and the
 * energy 1/2 sum_a Pw_a Jvec_a as the return value. */
double orc_exact_coulomb(int64_t M, const double* quat, const double* log_scale,
                         const double* centers, int64_t k, const double* C, const double* occ,
                         int64_t n, const int32_t* pi, const int32_t* pj, const double* weight,
                         double* J) {
    double tq[NQ], wq[NQ];
    node_table(tq, wq);
    Chart c = chart_alloc(M, quat, log_scale);
    PairRec* r = (PairRec*)malloc(sizeof(PairRec) * (n > 0 ? n : 1));
    double* Pw = (double*)malloc(sizeof(double) * (n > 0 ? n : 1));
    for (int64_t a = 0; a < n; ++a) {
        pair_rec(c.A9, centers, c.norm, pi[a], pj[a], r + a);
        Pw[a] = weight[a] * pair_density(k, C, occ, pi[a], pj[a]);
    }
#pragma omp parallel for schedule(dynamic, 16)
    for (int64_t a = 0; a < n; ++a) {
        double acc = 0.0;
        for (int64_t b = 0; b < n; ++b) {
            if (Pw[b] == 0.0) continue;
            acc += eri_schur_one(tq, wq, r + a, r + b) * Pw[b];
        }
        J[a] = acc;
    }
    double E = 0.0;
    for (int64_t a = 0; a < n; ++a) E += Pw[a] * J[a];
    free(Pw);
    free(r);
    chart_free(&c);
    return 0.5 * E;
}

