/* gsdft.h -- C ABI of the MI355X (gfx950) screened density-fitted Coulomb (DF-J) library.
 *
 * Every entry point takes device pointers, a caller-owned device workspace (size from the matching
 * *_workspace_size query) and a hipStream_t passed as void*. Kernels are enqueued on that stream;
 * an entry point returns before they finish unless its comment says it synchronises. Returns a
 * GSDFT_* status; gsdft_last_error() gives the message of the last failure on the calling thread.
 *
 * Layouts (all row-major, FP64 unless noted):
 *   quat (M,4) as (w,x,y,z), unnormalised; log_scale (M,3); centers (M,3);
 *   A6 (M,6) symmetric precision as xx,yy,zz,xy,xz,yz; norm (M);
 *   C (M,k); occ (k); pair list pi, pj (int32) and weight (n);
 *   aux log_alpha (N), aux_centers (N,3); metric V and its factor L (N,N) with L lower.
 *
 * Each declaration names the reference function it replaces (file:line in andresguzco/gs-dft).
 */
#ifndef GSDFT_H
#define GSDFT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GSDFT_OK 0
#define GSDFT_ERR_ARG 1          /* invalid argument (sizes, null pointers)                     */
#define GSDFT_ERR_OVERFLOW 2     /* significant pairs exceed twice the pad (pairs.py:157-161)   */
#define GSDFT_ERR_NOT_PD 3       /* Cholesky met a non-positive pivot                           */
#define GSDFT_ERR_HIP 4          /* HIP runtime error                                           */
#define GSDFT_ERR_LIB 5          /* hipCUB error                                                */
#define GSDFT_ERR_WORKSPACE 6    /* workspace too small; the query names the size               */
#define GSDFT_ERR_FALLBACK 7     /* spatial screening: the list overflows its pad (use the dense
                                    build) */

int gsdft_abi_version(void);
const char* gsdft_last_error(void);

/* Splat chart. Replaces Splat.A / Splat.norm, gs_dft/basis/spectral.py:33-40,72-82. */
int gsdft_splat_chart(int64_t M, const double* quat, const double* log_scale, double* A6,
                      double* norm, void* stream);

/* S_ij on a listed set of pairs. Replaces screened_overlap_pairs / _full_overlap_pairs,
 * gs_dft/screening/pairs.py:342-345,373-375. Workspace: gsdft_screen_workspace_size(M,0,0). */
int gsdft_overlap_pairs(int64_t M, const double* quat, const double* log_scale,
                        const double* centers, int64_t n, const int32_t* pi, const int32_t* pj,
                        double* S, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace for the screening calls. keep_cap = 0 for counting and for lists that fit their
 * pad; keep_cap >= n_sig for the keep-largest overflow path. */
int gsdft_screen_workspace_size(int64_t M, int unique, int64_t keep_cap, size_t* bytes);

/* Number of pairs with |S_ij| > eps (j >= i when unique). Replaces _count_significant,
 * gs_dft/screening/pairs.py:103-118. Synchronises the stream (one host read, as the reference's
 * int() at pairs.py:279). eps < 0 counts every pair without evaluating S. */
int gsdft_screen_count(int64_t M, const double* quat, const double* log_scale,
                       const double* centers, double eps, int unique, void* workspace,
                       size_t workspace_bytes, int64_t* n_sig, void* stream);

/* The padded pair list: lexsorted (ascending i*M+j), padding (0,0) with weight 0 at the tail,
 * weight 2 - delta_ij in unique mode and 1 otherwise. When n_sig > pad_to the pad_to largest |S|
 * are kept (ties by lower flat index) and re-sorted by flat index; beyond 2*pad_to the call fails
 * with GSDFT_ERR_OVERFLOW. If the overflow path needs a bigger workspace the call returns
 * GSDFT_ERR_WORKSPACE with *n_sig set. Synchronises the stream. Replaces neighbor_pairs,
 * _scan_flat_indices, _decode_flat, _keep_largest and _pair_weights,
 * gs_dft/screening/pairs.py:50-100,121-164,225-322. */
int gsdft_screen_build(int64_t M, const double* quat, const double* log_scale,
                       const double* centers, double eps, int unique, int64_t pad_to,
                       int32_t* pi, int32_t* pj, double* weight, void* workspace,
                       size_t workspace_bytes, int64_t* n_sig, void* stream);

/* Spatial screening: the same list as gsdft_screen_build when it fits the pad, built from a
 * candidate superset instead of every (i, j). A pair is a candidate when
 * |mu_i - mu_j|^2 < b_i + b_j, b_i = 1.0625 (-ln eps) / lmin_i with lmin_i a lower bound of the
 * smallest eigenvalue of A_i; every significant pair satisfies this (|S_ij| <= exp(-|d|^2 /
 * (1/lmin_i + 1/lmin_j))), so the result is bit-identical to the dense scan. pad_to < 0 only
 * counts (*n_sig). When n_sig > pad_to nothing is written and the call returns GSDFT_ERR_FALLBACK
 * with *n_sig set: the keep-largest list comes from gsdft_screen_build, as the reference falls
 * back to its dense strips. Needs eps >= 0 and M <= 262144 (one row's bitmap in LDS).
 * Synchronises the stream. Replaces _spatial_candidates and _scan_candidate_indices,
 * gs_dft/screening/pairs.py:167-222,284-298. */
int gsdft_screen_spatial_workspace_size(int64_t M, size_t* bytes);
int gsdft_screen_spatial(int64_t M, const double* quat, const double* log_scale,
                         const double* centers, double eps, int unique, int64_t pad_to,
                         int32_t* pi, int32_t* pj, double* weight, void* workspace,
                         size_t workspace_bytes, int64_t* n_sig, void* stream);

/* CSR views of the first n list entries for the atomics-free per-splat reductions of the
 * backward pass: row_ptr/row_perm group entries by pi, col_ptr/col_perm by pj, each group in list
 * order. row_ptr and col_ptr hold M+1 entries, the perms n. No reference counterpart: the
 * reference scatters with segment_sum inside JAX autodiff (gs_dft/coulomb/ri.py:436-469). */
int gsdft_pair_index_workspace_size(int64_t M, int64_t n, size_t* bytes);
int gsdft_pair_index(int64_t M, int64_t n, const int32_t* pi, const int32_t* pj,
                     int32_t* row_ptr, int32_t* row_perm, int32_t* col_ptr, int32_t* col_perm,
                     void* workspace, size_t workspace_bytes, void* stream);

/* Frozen diagonal product aux: log_alpha (n_scales*M) and centres, scale-major: one isotropic aux
 * per splat and scale at the self-product centre with exponent det(A_i + A_i)^(1/3) * scale.
 * scales is a HOST array of any length >= 1. The workspace is not used (pass NULL, 0). Replaces
 * init_product_aux(diagonal_only=True, or pi=None), gs_dft/basis/isotropic.py:81-116. */
int gsdft_product_aux(int64_t M, const double* quat, const double* log_scale,
                      const double* centers, const double* scales, int n_scales,
                      double* log_alpha, double* aux_centers, void* workspace,
                      size_t workspace_bytes, void* stream);

/* Frozen product aux of a listed set of pairs: log_alpha (n_scales*n) and centres, scale-major,
 * one aux per entry a at the product centre of (pi[a], pj[a]) with exponent
 * det(A_pi + A_pj)^(1/3) * scale, and exponent scale (alpha_0 = 1) where valid[a] == 0 (valid
 * may be NULL: every entry live). scales is a HOST array. Workspace:
 * gsdft_screen_workspace_size(M,0,0) (the charts). Replaces init_product_aux(basis, pi, pj, valid,
 * diagonal_only=False), gs_dft/basis/isotropic.py:106-116. */
int gsdft_product_aux_pairs(int64_t M, const double* quat, const double* log_scale,
                            const double* centers, int64_t n, const int32_t* pi,
                            const int32_t* pj, const double* valid, const double* scales,
                            int n_scales, double* log_alpha, double* aux_centers,
                            void* workspace, size_t workspace_bytes, void* stream);

/* Workspace for gsdft_aux_metric, gsdft_cholesky and gsdft_aux_cholesky. */
int gsdft_metric_workspace_size(int64_t N, size_t* bytes);

/* V_PQ = (P|Q) with lam added to the diagonal: the 1/r kernel for omega = 0, the long-range
 * kernel erf(omega r)/r for omega > 0 (ri.py:70-72); omega < 0, NaN or inf is refused. Replaces
 * aux_metric / coulomb_block / _coulomb_rows (+ shift_diag),
 * gs_dft/coulomb/ri.py:63-123,243-250,267-275. */
int gsdft_aux_metric(int64_t N, const double* log_alpha, const double* aux_centers, double lam,
                     double omega, double* V, void* workspace, size_t workspace_bytes,
                     void* stream);

/* In-place lower Cholesky of V (row-major), strict upper triangle zeroed. Synchronises the stream
 * to read the factorisation status. Replaces _chol_donated, gs_dft/coulomb/ri.py:253-256. */
int gsdft_cholesky(int64_t N, double* V, void* workspace, size_t workspace_bytes, void* stream);

/* L (N,N, row-major) = the lower Cholesky factor of V + lam I, V the metric gsdft_aux_metric forms
 * for the same arguments, strict upper triangle zero. Only the lower triangle of V is formed, in L's
 * own buffer, and factored in place. Synchronises the stream to read the factorisation status.
 * Replaces aux_cholesky, gs_dft/coulomb/ri.py:259-264. */
int gsdft_aux_cholesky(int64_t N, const double* log_alpha, const double* aux_centers, double lam,
                       double omega, double* L, void* workspace, size_t workspace_bytes,
                       void* stream);

/* d = (L L^T)^-1 gamma and, when energy is non-null, *energy = 0.5 gamma.d (device scalar).
 * Replaces df_coulomb_solve's cho_solve branch, gs_dft/coulomb/ri.py:472-479. */
int gsdft_cho_solve(int64_t N, const double* L, const double* gamma, double* d, double* energy,
                    void* stream);

/* gamma_P = sum_a (P|a) q_a over the first n list entries, q_a = w_a sum_o occ_o C_io C_jo.
 * Replaces df_coulomb_gamma_screened, gs_dft/coulomb/ri.py:436-469 (with full_isobra_block
 * :126-151 and the node kernel :167-185). */
int gsdft_gamma_workspace_size(int64_t M, int64_t k, int64_t N, int64_t n, size_t* bytes);
int gsdft_gamma(int64_t M, const double* quat, const double* log_scale, const double* centers,
                int64_t k, const double* C, const double* occ, int64_t N,
                const double* log_alpha, const double* aux_centers, int64_t n,
                const int32_t* pi, const int32_t* pj, const double* weight, double* gamma,
                void* workspace, size_t workspace_bytes, void* stream);

/* gsdft_gamma without a workspace and without allocating: the same kernels, with their scratch in
 * a static 64 MiB device array inside the library (one per GPU, held until the process ends; its
 * address is looked up once per device). No counterpart in the reference: it is for callers that
 * cannot allocate device memory (HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Sizes whose gsdft_gamma workspace exceeds 64 MiB (gsdft_gamma_workspace_size) are
 * refused with GSDFT_ERR_ARG before any launch: the water octamer (M = 600, N_aux = 2,400,
 * n = 166,915 pairs, 49.8 MiB) fits, C20H42 (n = 590,298, 179 MiB) does not.
 * Every call on one GPU shares that GPU's scratch and leaves its contents behind, so calls that
 * overlap on one GPU (several streams or host threads at once) race; serialise them. */
int gsdft_gamma_noalloc(int64_t M, const double* quat, const double* log_scale,
                        const double* centers, int64_t k, const double* C, const double* occ,
                        int64_t N, const double* log_alpha, const double* aux_centers, int64_t n,
                        const int32_t* pi, const int32_t* pj, const double* weight, double* gamma,
                        void* stream);

/* Reverse mode of gsdft_gamma for the cotangent dgamma (N), scaled by the device scalar
 * *dgamma_scale when non-null: J (n) = sum_P dgamma_P (P|a) (0 on zero-weight entries), and the
 * gradients w.r.t. quat, log_scale, centers (M,4/3/3) and C (M,k), aux held constant. Needs the
 * pair index of the same n entries. Replaces JAX's reverse pass through
 * gs_dft/coulomb/ri.py:436-469, :190-222, gs_dft/coulomb/stream.py:203-215 and
 * gs_dft/basis/spectral.py:33-40,72-82 (gs_dft/ks/train.py:367-373 holds the aux constant).
 * The pass is cut into slabs of at most 4096 aux functions, so that each slab's records stay in
 * one XCD's L2 while the workgroups running together walk it; the workspace holds 200 bytes per
 * pair for the slabs of one launch (all of them while that fits in 5 GiB, else as many as fit and
 * at least one, the launches adding their moments to running sums): 4.5 GB for 11.2 M pairs and
 * 80,000 aux functions, 4.1 GB for 20.6 M. */
int gsdft_gamma_vjp_workspace_size(int64_t M, int64_t k, int64_t N, int64_t n, size_t* bytes);
int gsdft_gamma_vjp(int64_t M, const double* quat, const double* log_scale,
                    const double* centers, int64_t k, const double* C, const double* occ,
                    int64_t N, const double* log_alpha, const double* aux_centers, int64_t n,
                    const int32_t* pi, const int32_t* pj, const double* weight,
                    const int32_t* row_ptr, const int32_t* row_perm, const int32_t* col_ptr,
                    const int32_t* col_perm, const double* dgamma, const double* dgamma_scale,
                    double* J, double* dquat, double* dlog_scale, double* dcenters, double* dC,
                    void* workspace, size_t workspace_bytes, void* stream);

/* out (n) = P_ij = sum_o occ_o C_io C_jo on the listed pairs. Replaces density_pairs,
 * gs_dft/screening/pairs.py:383-386. */
int gsdft_density_pairs(int64_t n, const int32_t* pi, const int32_t* pj, int64_t k,
                        const double* C, const double* occ, double* out, void* stream);

/* Nuclear attraction over the pair list. Workspace for both calls below. */
int gsdft_external_workspace_size(int64_t M, int64_t k, int64_t n, int64_t n_atoms,
                                  size_t* bytes);

/* V (n) = V_ij of every listed pair, -N_i N_j K sum_A Z_A (2/sqrt(pi)) sum_t w_t pi^1.5
 * det(B_t)^(-1/2) exp(...) with B_t = A_ij + t^2 I; atom_coords (n_atoms,3), atom_charges
 * (n_atoms). Replaces screened_nuclear_pairs / _full_nuclear_pairs,
 * gs_dft/screening/pairs.py:348-370,378-380. */
int gsdft_nuclear_pairs(int64_t M, const double* quat, const double* log_scale,
                        const double* centers, int64_t n, const int32_t* pi, const int32_t* pj,
                        int64_t n_atoms, const double* atom_coords, const double* atom_charges,
                        double* V, void* workspace, size_t workspace_bytes, void* stream);

/* *energy (device scalar) = sum_a w_a P_a V_a over the first n list entries, P_a = sum_o occ_o
 * C_io C_jo, and V (n) as gsdft_nuclear_pairs (0 on zero-weight entries). Optional outputs (null
 * to skip): the gradients w.r.t. quat, log_scale, centers and C (all four together, with the pair
 * index of the same n entries) and w.r.t. atom_coords (n_atoms,3). Replaces
 * screened_external_energy, gs_dft/screening/pairs.py:409-440, with
 * JAX's reverse pass through it (the only term gs_dft/ks/forces.py:53-77 differentiates in R). */
int gsdft_external_energy(int64_t M, const double* quat, const double* log_scale,
                          const double* centers, int64_t k, const double* C, const double* occ,
                          int64_t n, const int32_t* pi, const int32_t* pj, const double* weight,
                          const int32_t* row_ptr, const int32_t* row_perm,
                          const int32_t* col_ptr, const int32_t* col_perm, int64_t n_atoms,
                          const double* atom_coords, const double* atom_charges, double* energy,
                          double* V, double* dquat, double* dlog_scale, double* dcenters,
                          double* dC, double* datoms, void* workspace, size_t workspace_bytes,
                          void* stream);

/* Exact Hartree energy over the pair list (density-fitting free): *energy (device scalar) =
 * 1/2 sum_{a,b} (a|b) Pw_a Pw_b over the first n entries, Pw_a = w_a sum_o occ_o C_io C_jo, with
 * (a|b) the pair-pair Coulomb integral at the reference's 20-node rule, and J (n) = sum_b (a|b)
 * Pw_b (0 on zero-weight entries). Optional: the gradients w.r.t. quat, log_scale, centers and
 * C (all four, with the pair index of the same n entries; grads = 1 in the workspace query).
 * O(n^2) work. Replaces screened_coulomb_energy / full_eri_block_schur and JAX's reverse pass
 * through them, gs_dft/coulomb/stream.py:249-281,296-320 (ScreenedExactCoulomb,
 * gs_dft/ks/terms.py:193-205). */
int gsdft_exact_coulomb_workspace_size(int64_t M, int64_t k, int64_t n, int grads,
                                       size_t* bytes);
int gsdft_exact_coulomb(int64_t M, const double* quat, const double* log_scale,
                        const double* centers, int64_t k, const double* C, const double* occ,
                        int64_t n, const int32_t* pi, const int32_t* pj, const double* weight,
                        const int32_t* row_ptr, const int32_t* row_perm, const int32_t* col_ptr,
                        const int32_t* col_perm, double* energy, double* J, double* dquat,
                        double* dlog_scale, double* dcenters, double* dC, void* workspace,
                        size_t workspace_bytes, void* stream);

/* gsdft_exact_coulomb with the pair densities read from a density matrix: Pw_a = w_a P[i_a][j_a]
 * for P (M,M) row-major. Optional, each on its own: the splat gradients (dquat, dlog_scale,
 * dcenters together, with the pair index; grads = 1 in the workspace query) and dP (M,M) = dE/dP
 * = the Coulomb matrix on the listed entries, dP[i_a][j_a] = J_a and, for sym != 0 (a unique
 * list), dP[j_a][i_a] = J_a as well, zero elsewhere; the live entries must name distinct pairs.
 * Same workspace query as gsdft_exact_coulomb (k unused).
 * Replaces full_coulomb_energy / coulomb_energy_fused and its custom VJP,
 * gs_dft/coulomb/stream.py:127-187,284-287 (StreamedExactCoulomb, gs_dft/ks/terms.py:180-191),
 * over the list make_pairs builds (stream.py:47-60). */
int gsdft_exact_coulomb_density(int64_t M, const double* quat, const double* log_scale,
                                const double* centers, const double* P, int64_t n,
                                const int32_t* pi, const int32_t* pj, const double* weight,
                                int sym, const int32_t* row_ptr, const int32_t* row_perm,
                                const int32_t* col_ptr, const int32_t* col_perm, double* energy,
                                double* J, double* dquat, double* dlog_scale, double* dcenters,
                                double* dP, void* workspace, size_t workspace_bytes,
                                void* stream);

/* C (m x n, column-major, leading dimension ldc) = alpha op(A) op(B) + beta C in FP64 on the MFMA
 * units, op(X) = X for a zero trans flag and X^T otherwise, A and B column-major as in BLAS dgemm;
 * beta = 0 does not read C. No counterpart in the reference: the library's own dense product,
 * which the grid density and the exchange run on, exported so that it can be checked and timed
 * on its own. */
int gsdft_dgemm(int transa, int transb, int64_t m, int64_t n, int64_t k, double alpha,
                const double* A, int64_t lda, const double* B, int64_t ldb, double beta,
                double* C, int64_t ldc, void* stream);

/* Density on a grid for the exchange-correlation term, streamed over chunks of `chunk` points
 * (<= 65535): rho (G) and, for mode >= 1, grad (G,3), and for mode 2 tau (G), of the orbitals
 * C (M,k) with occupations occ at points (G,3). mode 0 replaces chunked_density, 1
 * chunked_density_and_grad, 2 chunked_density_grad_tau (gs_dft/screening/grid.py:60-70,88-154;
 * the dense eval_density_*_on_grid of gs_dft/integrals/dense.py give the same values). */
int gsdft_grid_density_workspace_size(int64_t M, int64_t k, int64_t chunk, int mode, int reverse,
                                      size_t* bytes);
int gsdft_grid_density(int64_t M, const double* quat, const double* log_scale,
                       const double* centers, int64_t k, const double* C, const double* occ,
                       int64_t G, const double* points, int64_t chunk, int mode, double* rho,
                       double* grad, double* tau, void* workspace, size_t workspace_bytes,
                       void* stream);

/* Reverse of gsdft_grid_density for the cotangents v_rho (G), v_grad (G,3), v_tau (G) (null =
 * zero): the gradients w.r.t. quat, log_scale, centers (M,4/3/3) and C (M,k); the points are held
 * constant. Workspace query with reverse = 1. Replaces JAX's reverse pass through
 * gs_dft/screening/grid.py:88-154. */
int gsdft_grid_density_vjp(int64_t M, const double* quat, const double* log_scale,
                           const double* centers, int64_t k, const double* C, const double* occ,
                           int64_t G, const double* points, int64_t chunk, int mode,
                           const double* v_rho, const double* v_grad, const double* v_tau,
                           double* dquat, double* dlog_scale, double* dcenters, double* dC,
                           void* workspace, size_t workspace_bytes, void* stream);

/* Screened exact exchange through density fitting (RI-K): E_K = -Tr((V + lam I)^-1 M) with
 * M_PQ = sum_oo' D[P,o,o'] D[Q,o,o'] and D[P,o,o'] = sum over the first n listed pairs
 * a = (pi[a], pj[a]) of weight[a] C_io C_ko' (P|a) (weight null: all 1). The reference passes the
 * ordered list with 0/1 weights and reads them as a mask (ri.py:509-520); other weights multiply
 * their entries here, an integer weight w counting as the entry listed w times. Replaces
 * gs_dft/coulomb/ri.py:497-544 (df_exchange_energy_screened and _exchange_M_streamed_screened) as
 * called from gs_dft/ks/terms.py:250-253 with the frozen
 * product aux (N functions: log_alpha, aux_centers) and chol = the row-major lower Cholesky factor
 * of V + lam I (gsdft_cholesky). C is the (M, k) occupied block (occupation 2 folded into the
 * prefactor, as in the reference). row_ptr/row_perm (and col_ptr/col_perm for gradients) are the
 * CSR index of the list (gsdft_pair_index). symmetric = 1 asserts that every live entry (i, j, w)
 * has its (j, i, w): D_P is then symmetric and only its k(k+1)/2 symmetric columns are solved
 * (the antisymmetric part is round-off); with 0 all k^2 columns are kept. aux_chunk = aux
 * functions per pass (0: the library's choice; the result does not depend on it beyond
 * round-off). With gradients the forward keeps its (M, N, k) products for the reverse when they
 * fit in 32 GiB; recompute = 1 forgoes that and recomputes them (less memory, more time), the
 * role the reference's occ_chunk knob plays for its memory. omega = 0 is exchange with 1/r;
 * omega > 0 is the long-range exchange E_K[erf(omega r)/r] of range-separated hybrids
 * (gs_dft/ks/terms.py:258-264): the three-centre integrals then use the 12-node Gauss-Legendre rule
 * on [0, omega] (ri.py:231-235) and chol must factor the erf metric (gsdft_aux_metric with the
 * same omega). Entries of one unordered splat pair with equal weights ((i, j) and (j, i), repeats
 * included) share their product Gaussian, so each (P|a) is formed once per such pair and serves
 * all its entries (the result equals the entry-by-entry sum to round-off). The call never waits
 * on the host (the stream's work is only queued). Writes energy (one device double); with
 * non-null dquat also dE_K/d(quat, log_scale, centers, C) (M x 4, 3, 3, k). */
int gsdft_exchange_workspace_size(int64_t M, int64_t k, int64_t N, int64_t n, int symmetric,
                                  int grads, int64_t aux_chunk, int recompute, size_t* bytes);
int gsdft_exchange(int64_t M, const double* quat, const double* log_scale, const double* centers,
                   int64_t k, const double* C, int64_t N, const double* log_alpha,
                   const double* aux_centers, const double* chol, int64_t n, const int32_t* pi,
                   const int32_t* pj, const double* weight, const int32_t* row_ptr,
                   const int32_t* row_perm, const int32_t* col_ptr, const int32_t* col_perm,
                   int symmetric, int64_t aux_chunk, int recompute, double omega,
                   double* energy, double* dquat,
                   double* dlog_scale, double* dcenters, double* dC, void* workspace,
                   size_t workspace_bytes, void* stream);

/* Kernel timing with HIP events on the launch stream (no reference counterpart). Ids:
 * 0 three-centre forward, 1 three-centre reverse, 2 screening, 3 metric, 4 Cholesky, 5 solve,
 * 6 nuclear attraction per pair (values, splat moments and, with nuclear gradients, each pair
 * block's forces on the nuclei), 7 nuclear attraction per nucleus (the fixed-order force sums),
 * 8 exact pair-pair Coulomb (values), 9 exact pair-pair Coulomb (values and gradient moments),
 * 10 exchange three-centre block, 11 exchange three-centre reverse, 12 exchange triangular
 * solves (blocked, FP64 MFMA), 13 exchange GEMMs (FP64 MFMA), 14 exchange pair-sparse products (Y = T C and
 * the sampled Tbar). gsdft_profile_read synchronises the recorded events and returns the summed
 * milliseconds and the launch count since the last reset. gsdft_profile_read_work returns the
 * work units the kernels executed while profiling was on (ids 0, 1, 6-11: quadrature nodes
 * evaluated, summed over live lanes, so at most 20 x (aux functions, nuclei or pairs) x pairs
 * per launch; other ids: 0). Profiling allocates a few bytes of device memory on the device
 * current when it is first enabled. */
int gsdft_profile_enable(int on);
int gsdft_profile_read(int id, double* total_ms, int64_t* launches, int reset);
int gsdft_profile_read_work(int id, uint64_t* units, int reset);

#ifdef __cplusplus
}
#endif
#endif
