/* CPU oracle for the screened density-fitted Coulomb (DF-J) path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C FP64 restatement of the reference JAX algorithm,
 * used as the parity checker for the HIP path and as the CPU baseline in the benchmark. Nothing in
 * the shipped library links, loads or calls it.
 *
 * Conventions: all matrices are row-major. Per-splat 3x3 precisions are stored as full 9-entry
 * matrices, as the reference holds them. Pair indices are int32 (the reference decodes its int64
 * flat indices to int32 pi/pj). All arrays are host memory. Status codes: 0 ok, nonzero error.
 */
#ifndef GSDFT_ORACLE_H
#define GSDFT_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* gs_dft/integrals/dense.py:46-53,77 -- the 20-node half-line Gauss-Legendre table, filled by
 * Newton iteration on P_20 (independent of numpy's leggauss). */
void orc_quad_table(int n, double* t, double* w);

/* Install the 20-node table used by the three-centre routines (t, w: 20 doubles each). */
void orc_set_quad_table(const double* t, const double* w);

/* gs_dft/basis/spectral.py:33-40,72-82 -- chart: A (M,9) and N (M). */
void orc_chart(int64_t M, const double* quat, const double* log_scale, double* A9, double* norm);

/* gs_dft/coulomb/stream.py:203-215 -- product precision (n,9), centre (n,3), N_iN_jK (n). */
void orc_pair_quantities(int64_t M, const double* A9, const double* mu, const double* norm,
                         int64_t n, const int32_t* pi, const int32_t* pj,
                         double* Ah9, double* Pc, double* KN);

/* gs_dft/screening/pairs.py:342-345 -- S_ij for listed pairs. */
void orc_overlap_pairs(int64_t M, const double* quat, const double* log_scale,
                       const double* centers, int64_t n, const int32_t* pi, const int32_t* pj,
                       double* S);

/* gs_dft/screening/pairs.py:103-118 -- number of |S_ij| > eps (j >= i when unique). */
int64_t orc_count_significant(int64_t M, const double* quat, const double* log_scale,
                              const double* centers, double eps, int unique);

/* gs_dft/screening/pairs.py:225-322 -- the padded, lexsorted pair list.
 * pad_to < 0 means "no pad": the list is sized to the significant count, which the caller must
 * have allocated (query it with orc_count_significant). On return *n_out holds the list length
 * and *n_sig the significant count. Returns 0, or 2 when n_sig exceeds twice the pad (the
 * reference raises ValueError there). weight: (2 - delta_ij) for unique, 1 for ordered, 0 on the
 * padding. */
int orc_neighbor_pairs(int64_t M, const double* quat, const double* log_scale,
                       const double* centers, double eps, int64_t pad_to, int unique,
                       int32_t* pi, int32_t* pj, double* weight, int64_t* n_out, int64_t* n_sig);

/* Knife-edge audit: candidates with ||S| - eps| <= rel_tol eps, and min ||S| - eps| / eps. */
void orc_screen_margin(int64_t M, const double* quat, const double* log_scale,
                       const double* centers, double eps, int unique, double rel_tol,
                       int64_t* n_close, double* min_gap);

/* gs_dft/screening/pairs.py:167-197 (+ grid.py:76-82) -- the spatial candidate rules checked
 * against the significant set by brute force (see oracle.c). */
void orc_spatial_audit(int64_t M, const double* quat, const double* log_scale,
                       const double* centers, double eps, int unique, double safety,
                       int64_t* n_sig, int64_t* n_cand_ref, int64_t* n_miss_ref,
                       int64_t* n_cand_bound, int64_t* n_miss_bound, double* max_ratio);

/* gs_dft/basis/isotropic.py:81-116 -- diagonal product aux: log_alpha (S*M), centres (S*M,3),
 * scale-major. */
void orc_product_aux(int64_t M, const double* quat, const double* log_scale,
                     const double* centers, const double* scales, int n_scales,
                     double* log_alpha, double* aux_centers);

/* gs_dft/basis/isotropic.py:106-116 -- product aux of listed pairs (diagonal_only=False):
 * log_alpha (S*n), centres (S*n,3), scale-major; alpha_0 = 1 where valid[a] == 0 (valid may be
 * NULL). */
void orc_product_aux_pairs(int64_t M, const double* quat, const double* log_scale,
                           const double* centers, int64_t n, const int32_t* pi,
                           const int32_t* pj, const double* valid, const double* scales,
                           int n_scales, double* log_alpha, double* aux_centers);

/* gs_dft/coulomb/ri.py:63-76,267-275 (+ shift_diag :243-250 when lam != 0) -- metric V (N,N);
 * omega != 0 selects the kernel erf(omega r)/r (ri.py:70-72). */
void orc_aux_metric(int64_t N, const double* log_alpha, const double* centers, double lam,
                    double omega, double* V);

/* Rows `rows` (nrows of them) of the metric orc_aux_metric forms: V (nrows, N). */
void orc_aux_metric_rows(int64_t N, const double* log_alpha, const double* centers, double lam,
                         double omega, int64_t nrows, const int64_t* rows, double* V);

/* Boys F0 used by the metric: 0.5*sqrt(pi/T)*erf(sqrt(T)), series below 1e-12. */
double orc_boys0(double T);

/* gs_dft/coulomb/ri.py:253-264 -- in-place lower Cholesky (row-major), strict upper zeroed.
 * Returns 0, or 1 when a pivot is not positive. */
int orc_cholesky(int64_t N, double* V);

/* gs_dft/coulomb/ri.py:479 -- cho_solve((L, lower), gamma). */
void orc_cho_solve(int64_t N, const double* L, const double* gamma, double* d);

/* gs_dft/coulomb/ri.py:126-151,167-185 -- (P|a) block for listed pairs, (N, n) row-major. */
void orc_three_center_block(int64_t M, const double* quat, const double* log_scale,
                            const double* centers, int64_t N, const double* log_alpha,
                            const double* aux_centers, int64_t n, const int32_t* pi,
                            const int32_t* pj, double* block);

/* gs_dft/coulomb/ri.py:436-469 -- gamma (N). */
void orc_gamma(int64_t M, const double* quat, const double* log_scale, const double* centers,
               int64_t k, const double* C, const double* occ, int64_t N,
               const double* log_alpha, const double* aux_centers, int64_t n,
               const int32_t* pi, const int32_t* pj, const double* weight, double* gamma);

/* Reverse mode of orc_gamma for an upstream dgamma (N): J (n) = sum_P dgamma_P (P|a), and the
 * gradients w.r.t. quat (M,4), log_scale (M,3), centers (M,3) and C (M,k). The aux is held
 * constant, as the reference holds the refresh state constant (gs_dft/ks/train.py:367-373). */
void orc_gamma_vjp(int64_t M, const double* quat, const double* log_scale, const double* centers,
                   int64_t k, const double* C, const double* occ, int64_t N,
                   const double* log_alpha, const double* aux_centers, int64_t n,
                   const int32_t* pi, const int32_t* pj, const double* weight,
                   const double* dgamma, double* J, double* dquat, double* dlog_scale,
                   double* dcenters, double* dC);

/* V (n) of gs_dft/screening/pairs.py:348-370 for the listed pairs and nuclei (coords (n_atoms,3),
 * charges (n_atoms)), in the reference's B = A + t^2 I form. */
void orc_nuclear_pairs(int64_t M, const double* quat, const double* log_scale,
                       const double* centers, int64_t n, const int32_t* pi, const int32_t* pj,
                       int64_t n_atoms, const double* coords, const double* charges, double* V);

/* E_ext = sum_a w_a P_a V_a (gs_dft/screening/pairs.py:409-440). */
double orc_external_energy(int64_t M, const double* quat, const double* log_scale,
                           const double* centers, int64_t k, const double* C, const double* occ,
                           int64_t n, const int32_t* pi, const int32_t* pj, const double* weight,
                           int64_t n_atoms, const double* coords, const double* charges);

/* (a|b) of gs_dft/coulomb/stream.py:249-281 for bra pairs (ai, aj) x ket pairs (bi, bj), row-major
 * (na, nb), in the reference's Schur-complement node form. */
void orc_eri_block(int64_t M, const double* quat, const double* log_scale, const double* centers,
                   int64_t na, const int32_t* ai, const int32_t* aj, int64_t nb,
                   const int32_t* bi, const int32_t* bj, double* out);

/* J (n) = sum_b (a|b) Pw_b over the list; returns E_J = 1/2 sum_a Pw_a J_a
 * (gs_dft/coulomb/stream.py:296-320). */
double orc_exact_coulomb(int64_t M, const double* quat, const double* log_scale,
                         const double* centers, int64_t k, const double* C, const double* occ,
                         int64_t n, const int32_t* pi, const int32_t* pj, const double* weight,
                         double* J);

/* The worker count the OpenMP loops above use (1 when built without OpenMP). */
int orc_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
