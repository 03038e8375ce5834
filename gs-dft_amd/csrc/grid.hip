// Density on a grid for the exchange-correlation term: rho, grad rho and tau of the splat
// orbitals at grid points, and their reverse pass (gs_dft/screening/grid.py:60-70,88-140).
//
// Per chunk of Gc grid points (rows):
//   g_rm = N_m exp(-dr.A_m dr), dg_rm = -2 A_m dr g_rm      (k_grid_basis, VALU, one lane per (r,m))
//   psi = g C, dpsi_d = dg_d C                              (FP64 MFMA products, gemm.hip)
//   rho_r = sum_o occ_o psi_ro^2
//   grad rho_r = 2 sum_m phi_rm dg_rm, phi = (psi occ) C^T   (grid.py:104-107; the tau variant
//                uses 2 sum_o occ_o psi_ro dpsi_ro as grid.py:132 does)
//   tau_r = 1/2 sum_o occ_o |dpsi_ro|^2
// Reverse, for cotangents (v_rho, v_grad, v_tau):
//   Pbar   = 2 v_rho occ psi + 2 occ sum_d v_grad,d dpsi_d,  Pbar_d = 2 occ v_grad,d psi + v_tau occ dpsi_d
//   dC    += [g; dg]^T [Pbar; Pbar_d]                       (one GEMM over the stacked rows)
//   [gbar; dgbar] = [Pbar; Pbar_d] C^T                      (one GEMM)
//   then per (r, m) the basis reverse, summed over rows per splat in fixed order, and the chart
//   reverse. No atomics; the result does not depend on the chunk size beyond round-off of the
//   row order inside the GEMMs.
//
// Storage: row-major (Gc, M) basis blocks (the column-major (M, Gc) view the products read),
// row-major (Gc, k) orbital blocks with rows ldk = k + (k & 1) doubles apart; g and the three dg
// blocks are consecutive, as are psi and the dpsi. The even row length keeps every operand of the
// products 16-byte aligned row by row, which their LDS-DMA path needs; for odd k the products read
// C from a copy with rows of ldk (the last column zero).
#include "common.h"
#include "internal.h"

namespace gsdft {

namespace {

inline unsigned nblk(int64_t n, int bs) { return (unsigned)((n + bs - 1) / bs); }

// One lane per (row r, splat m): grid (ceil(M/256), Gc).
__global__ __launch_bounds__(256) void k_grid_basis(int64_t M, int64_t Gc,
                                                    const double* __restrict__ pts,
                                                    const double* __restrict__ A6,
                                                    const double* __restrict__ mu,
                                                    const double* __restrict__ Nrm,
                                                    double* __restrict__ g,
                                                    double* __restrict__ dg) {
    const int64_t m = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    const int64_t r = blockIdx.y;
    if (m >= M) return;
    const double dx = pts[3 * r] - mu[3 * m], dy = pts[3 * r + 1] - mu[3 * m + 1],
                 dz = pts[3 * r + 2] - mu[3 * m + 2];
    const double* a = A6 + 6 * m;
    const double u0 = a[0] * dx + a[3] * dy + a[4] * dz;     // (A dr), grid.py:60-66
    const double u1 = a[3] * dx + a[1] * dy + a[5] * dz;
    const double u2 = a[4] * dx + a[5] * dy + a[2] * dz;
    const double gv = Nrm[m] * exp(-(dx * u0 + dy * u1 + dz * u2));
    g[r * M + m] = gv;
    if (dg) {
        dg[r * M + m] = -2.0 * u0 * gv;
        dg[(Gc + r) * M + m] = -2.0 * u1 * gv;
        dg[(2 * Gc + r) * M + m] = -2.0 * u2 * gv;
    }
}

// Cp[m ldk + o] = C[m k + o] for o < k, 0 for k <= o < ldk.
__global__ void k_grid_pad_cols(int64_t M, int64_t k, int64_t ldk, const double* __restrict__ C,
                                double* __restrict__ Cp) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= M * ldk) return;
    const int64_t m = i / ldk, o = i % ldk;
    Cp[i] = o < k ? C[m * k + o] : 0.0;
}

// rho_r = sum_o occ_o psi_ro^2, one wave per row.
__global__ __launch_bounds__(256) void k_grid_rho(int64_t Gc, int64_t k, int64_t ldk,
                                                  const double* __restrict__ psi,
                                                  const double* __restrict__ occ,
                                                  double* __restrict__ rho) {
    const int64_t r = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (r >= Gc) return;
    double s = 0.0;
    for (int64_t o = lane; o < k; o += 64) {
        const double p = psi[r * ldk + o];
        s = __builtin_fma(occ[o] * p, p, s);
    }
    s = wave_sum(s);
    if (lane == 0) rho[r] = s;
}

// out = psi * occ (column scaling of the (Gc, k) block, rows ldk apart).
__global__ void k_grid_scale_occ(int64_t Gc, int64_t k, int64_t ldk,
                                 const double* __restrict__ psi, const double* __restrict__ occ,
                                 double* __restrict__ out) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= Gc * k) return;
    const int64_t e = (i / k) * ldk + i % k;
    out[e] = psi[e] * occ[i % k];
}

// grad_rd = 2 sum_m phi_rm dg_d,rm, one wave per row (grid.py:104-107).
__global__ __launch_bounds__(256) void k_grid_grad_phi(int64_t Gc, int64_t M,
                                                       const double* __restrict__ phi,
                                                       const double* __restrict__ dg,
                                                       double* __restrict__ grad) {
    const int64_t r = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (r >= Gc) return;
    double s0 = 0.0, s1 = 0.0, s2 = 0.0;
    for (int64_t m = lane; m < M; m += 64) {
        const double f = phi[r * M + m];
        s0 = __builtin_fma(f, dg[r * M + m], s0);
        s1 = __builtin_fma(f, dg[(Gc + r) * M + m], s1);
        s2 = __builtin_fma(f, dg[(2 * Gc + r) * M + m], s2);
    }
    s0 = wave_sum(s0); s1 = wave_sum(s1); s2 = wave_sum(s2);
    if (lane == 0) {
        grad[3 * r] = 2.0 * s0;
        grad[3 * r + 1] = 2.0 * s1;
        grad[3 * r + 2] = 2.0 * s2;
    }
}

// grad_rd = 2 sum_o occ_o psi_ro dpsi_d,ro and tau_r = 1/2 sum_o occ_o |dpsi_ro|^2 (grid.py:128-134).
__global__ __launch_bounds__(256) void k_grid_grad_tau(int64_t Gc, int64_t k, int64_t ldk,
                                                       const double* __restrict__ psi,
                                                       const double* __restrict__ occ,
                                                       double* __restrict__ grad,
                                                       double* __restrict__ tau) {
    const int64_t r = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (r >= Gc) return;
    const double* dpsi = psi + Gc * ldk;
    double s0 = 0.0, s1 = 0.0, s2 = 0.0, t = 0.0;
    for (int64_t o = lane; o < k; o += 64) {
        const double op = occ[o] * psi[r * ldk + o];
        const double d0 = dpsi[r * ldk + o], d1 = dpsi[(Gc + r) * ldk + o],
                     d2 = dpsi[(2 * Gc + r) * ldk + o];
        s0 = __builtin_fma(op, d0, s0);
        s1 = __builtin_fma(op, d1, s1);
        s2 = __builtin_fma(op, d2, s2);
        t = __builtin_fma(occ[o], __builtin_fma(d0, d0, __builtin_fma(d1, d1, d2 * d2)), t);
    }
    s0 = wave_sum(s0); s1 = wave_sum(s1); s2 = wave_sum(s2); t = wave_sum(t);
    if (lane == 0) {
        grad[3 * r] = 2.0 * s0;
        grad[3 * r + 1] = 2.0 * s1;
        grad[3 * r + 2] = 2.0 * s2;
        if (tau) tau[r] = 0.5 * t;
    }
}

// Pbar = 2 v_rho occ psi + 2 occ sum_d v_grad,d dpsi_d; Pbar_d = 2 occ v_grad,d psi
// + v_tau occ dpsi_d. One lane per (r, o); psi and dpsi consecutive (Gc, k) blocks with rows ldk
// apart, likewise pbar.
__global__ void k_grid_pbar(int64_t Gc, int64_t k, int64_t ldk, int mode,
                            const double* __restrict__ psi, const double* __restrict__ occ,
                            const double* __restrict__ v_rho, const double* __restrict__ v_grad,
                            const double* __restrict__ v_tau, double* __restrict__ pbar) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= Gc * k) return;
    const int64_t r = i / k, o = i % k, e = r * ldk + o;
    const double oc = occ[o], p = psi[e];
    double pb = 2.0 * (v_rho ? v_rho[r] : 0.0) * oc * p;
    if (mode >= 1) {
        const double* dpsi = psi + Gc * ldk;
        const double vg[3] = {v_grad ? v_grad[3 * r] : 0.0, v_grad ? v_grad[3 * r + 1] : 0.0,
                              v_grad ? v_grad[3 * r + 2] : 0.0};
        const double vt = (mode == 2 && v_tau) ? v_tau[r] : 0.0;
#pragma unroll
        for (int d = 0; d < 3; ++d) {
            const double dp = dpsi[d * Gc * ldk + e];
            pb = __builtin_fma(2.0 * oc * vg[d], dp, pb);
            pbar[(1 + d) * Gc * ldk + e] = __builtin_fma(2.0 * oc * vg[d], p, vt * oc * dp);
        }
    }
    pbar[e] = pb;
}

// Basis reverse for splat m over the rows [r0, r1) of the chunk, added to partial[slab][c][m]:
//   G_g = gbar - 2 sum_d dgbar_d u_d, U_d = -2 g dgbar_d, c = -G_g g (= dE/dq, q = dr.A dr),
//   dE/dA += c dr dr^T + sym(U dr^T), dE/dmu -= 2 c u + A U, dE/dN += G_g g / N.
__global__ __launch_bounds__(256) void k_grid_basis_bwd(
    int64_t M, int64_t Gc, int64_t rows_per_slab, const double* __restrict__ pts,
    const double* __restrict__ A6, const double* __restrict__ mu, const double* __restrict__ Nrm,
    const double* __restrict__ g, const double* __restrict__ gbar, int mode,
    double* __restrict__ partial) {
    const int64_t m = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (m >= M) return;
    const int64_t r0 = blockIdx.y * rows_per_slab;
    const int64_t r1 = min(Gc, r0 + rows_per_slab);
    const double* a = A6 + 6 * m;
    const double mx = mu[3 * m], my = mu[3 * m + 1], mz = mu[3 * m + 2];
    double acc[10] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t r = r0; r < r1; ++r) {
        const double dr[3] = {pts[3 * r] - mx, pts[3 * r + 1] - my, pts[3 * r + 2] - mz};
        const double u[3] = {a[0] * dr[0] + a[3] * dr[1] + a[4] * dr[2],
                             a[3] * dr[0] + a[1] * dr[1] + a[5] * dr[2],
                             a[4] * dr[0] + a[5] * dr[1] + a[2] * dr[2]};
        const double gv = g[r * M + m];
        double Gg = gbar[r * M + m];
        double U[3] = {0.0, 0.0, 0.0};
        if (mode >= 1) {
#pragma unroll
            for (int d = 0; d < 3; ++d) {
                const double db = gbar[((1 + d) * Gc + r) * M + m];
                Gg = __builtin_fma(-2.0 * db, u[d], Gg);
                U[d] = -2.0 * gv * db;
            }
        }
        const double c = -Gg * gv;
        acc[0] += c * dr[0] * dr[0] + U[0] * dr[0];
        acc[1] += c * dr[1] * dr[1] + U[1] * dr[1];
        acc[2] += c * dr[2] * dr[2] + U[2] * dr[2];
        acc[3] += c * dr[0] * dr[1] + 0.5 * (U[0] * dr[1] + dr[0] * U[1]);
        acc[4] += c * dr[0] * dr[2] + 0.5 * (U[0] * dr[2] + dr[0] * U[2]);
        acc[5] += c * dr[1] * dr[2] + 0.5 * (U[1] * dr[2] + dr[1] * U[2]);
        const double AU[3] = {a[0] * U[0] + a[3] * U[1] + a[4] * U[2],
                              a[3] * U[0] + a[1] * U[1] + a[5] * U[2],
                              a[4] * U[0] + a[5] * U[1] + a[2] * U[2]};
        acc[6] -= 2.0 * c * u[0] + AU[0];
        acc[7] -= 2.0 * c * u[1] + AU[1];
        acc[8] -= 2.0 * c * u[2] + AU[2];
        acc[9] += Gg * gv;                               // divided by N below
    }
    acc[9] /= Nrm[m];
    double* o = partial + (int64_t)blockIdx.y * 10 * M + m;
#pragma unroll
    for (int c = 0; c < 10; ++c) o[(int64_t)c * M] += acc[c];
}

// Per splat: sum the slab partials in fixed order, then the chart reverse.
__global__ void k_grid_splat_grad(int64_t M, int64_t slabs, const double* __restrict__ partial,
                                  const double* __restrict__ quat,
                                  const double* __restrict__ log_scale,
                                  double* __restrict__ dquat, double* __restrict__ dlog_scale,
                                  double* __restrict__ dcenters) {
    const int64_t m = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (m >= M) return;
    double acc[10];
    for (int c = 0; c < 10; ++c) {
        double s = 0.0;
        for (int64_t k = 0; k < slabs; ++k) s += partial[(k * 10 + c) * M + m];
        acc[c] = s;
    }
    chart_reverse(m, acc, quat, log_scale, dquat, dlog_scale, dcenters);
}

__global__ void k_grid_fill(int64_t n, double v, double* __restrict__ out) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i < n) out[i] = v;
}

constexpr int64_t kRowsPerSlab = 64;

// Row length of the orbital blocks (even: every row of the products' operands 16-byte aligned).
inline int64_t grid_ldk(int64_t k) { return k + (k & 1); }

struct GridWs {
    double *A6, *Nrm, *gb, *pb, *phi, *gbar, *pbar, *partial;
    double* Cp;               // C with rows of grid_ldk(k) (odd k only)
    double* part;             // K slices of the products with few output tiles (gemm_cm_split)
    int64_t part_doubles;
};

int layout_grid(Arena& ar, int64_t M, int64_t k, int64_t chunk, int mode, bool reverse,
                GridWs* w) {
    const int nb = mode >= 1 ? 4 : 1;
    const int64_t ldk = grid_ldk(k);
    w->A6 = ar.take<double>(6 * M + 1);
    w->Nrm = ar.take<double>(M + 1);
    w->gb = ar.take<double>(nb * chunk * M + 1);
    w->pb = ar.take<double>(nb * chunk * ldk + 1);
    w->phi = (!reverse && mode == 1) ? ar.take<double>(chunk * M + 1) : nullptr;
    w->gbar = reverse ? ar.take<double>(nb * chunk * M + 1) : nullptr;
    w->pbar = reverse ? ar.take<double>(nb * chunk * ldk + 1) : nullptr;
    w->Cp = ldk != k ? ar.take<double>(M * ldk + 1) : nullptr;
    const int64_t slabs = (chunk + kRowsPerSlab - 1) / kRowsPerSlab;
    w->partial = reverse ? ar.take<double>(slabs * 10 * M + 1) : nullptr;
    // room for the slices of the orbital product (k x nb chunk over K = M) and, in the reverse,
    // of dC (k x M over K = nb chunk) at the chunk's full size; smaller chunks split into at most
    // as many blocks of their own size as fit
    const int64_t orb = gemm_split_slices(k, nb * chunk, M) * k * nb * chunk;
    const int64_t dc = reverse ? gemm_split_slices(k, M, nb * chunk) * k * M : 0;
    w->part_doubles = std::max<int64_t>(orb > k * nb * chunk ? orb : 0, dc > k * M ? dc : 0);
    w->part = w->part_doubles > 0 ? ar.take<double>(w->part_doubles) : nullptr;
    return GSDFT_OK;
}

// C as the products read it: rows of grid_ldk(k) (a padded copy for odd k).
int grid_c(int64_t M, int64_t k, const double* C, const GridWs& w, hipStream_t s,
           const double** Cuse) {
    const int64_t ldk = grid_ldk(k);
    if (ldk == k) {
        *Cuse = C;
        return GSDFT_OK;
    }
    k_grid_pad_cols<<<nblk(M * ldk, 256), 256, 0, s>>>(M, k, ldk, C, w.Cp);
    GSDFT_HIP(hipGetLastError());
    *Cuse = w.Cp;
    return GSDFT_OK;
}

int check_grid_args(int64_t M, int64_t k, int64_t G, int64_t chunk, int mode) {
    if (M <= 0 || k <= 0 || G < 0 || chunk <= 0 || chunk > 65535 || mode < 0 || mode > 2)
        return fail(GSDFT_ERR_ARG, "grid density: need M, k > 0, G >= 0, 0 < chunk <= 65535 and "
                    "mode 0 (rho), 1 (rho, grad) or 2 (rho, grad, tau)");
    GSDFT_TRY(check_items(M * (k + 1), "grid density", "the orbitals (M x k)"));
    GSDFT_TRY(check_items(chunk * (k + 1), "grid density", "a chunk's orbital values"));
    GSDFT_TRY(check_items(((chunk + kRowsPerSlab - 1) / kRowsPerSlab) * 10 * M, "grid density",
                          "the reverse's per-slab moments"));
    return GSDFT_OK;
}

// psi (and dpsi) for rows [0, Gc) of the chunk: [psi; dpsi] (nb Gc x k) = [g; dg] (nb Gc x M) C,
// C (from grid_c) and the result with rows of grid_ldk(k).
int grid_orbitals(int64_t M, int64_t k, int64_t Gc, int nb, const double* Cuse, const double* gb,
                  double* pb, const GridWs& w, hipStream_t s) {
    const int64_t ldk = grid_ldk(k);
    // column-major: pb (k x nb Gc, leading dimension ldk) = C^T-view (k x M) * gb (M x nb Gc)
    return gemm_cm_split('N', 'N', k, nb * Gc, M, 1.0, Cuse, ldk, gb, M, 0.0, pb, ldk, w.part,
                         w.part_doubles, s);
}

}  // namespace

}  // namespace gsdft

using namespace gsdft;

extern "C" int gsdft_grid_density_workspace_size(int64_t M, int64_t k, int64_t chunk, int mode,
                                                 int reverse, size_t* bytes) {
    if (!bytes) return fail(GSDFT_ERR_ARG, "grid_density_workspace_size: null output");
    GSDFT_TRY(check_grid_args(M, k, 0, chunk, mode));
    Arena ar{nullptr, 0, 0};
    GridWs w;
    GSDFT_TRY(layout_grid(ar, M, k, chunk, mode, reverse != 0, &w));
    *bytes = ar.need();
    return GSDFT_OK;
}

extern "C" int gsdft_grid_density(int64_t M, const double* quat, const double* log_scale,
                                  const double* centers, int64_t k, const double* C,
                                  const double* occ, int64_t G, const double* points,
                                  int64_t chunk, int mode, double* rho, double* grad, double* tau,
                                  void* workspace, size_t workspace_bytes, void* stream) {
    GSDFT_TRY(check_grid_args(M, k, G, chunk, mode));
    if (!quat || !log_scale || !centers || !C || !occ || (G > 0 && (!points || !rho)) ||
        (mode >= 1 && G > 0 && !grad) || (mode == 2 && G > 0 && !tau))
        return fail(GSDFT_ERR_ARG, "gsdft_grid_density: null argument");
    if (G == 0) return GSDFT_OK;
    hipStream_t s = (hipStream_t)stream;
    Arena ar{(char*)workspace, workspace_bytes, 0};
    GridWs w;
    GSDFT_TRY(layout_grid(ar, M, k, chunk, mode, false, &w));
    if (!w.pb || (mode == 1 && !w.phi) || (w.part_doubles > 0 && !w.part) ||
        (grid_ldk(k) != k && !w.Cp))
        return fail(GSDFT_ERR_WORKSPACE, "gsdft_grid_density: workspace too small");
    const int64_t ldk = grid_ldk(k);
    const double* Cuse = nullptr;
    GSDFT_TRY(grid_c(M, k, C, w, s, &Cuse));
    GSDFT_TRY(launch_chart(M, quat, log_scale, w.A6, w.Nrm, s));
    for (int64_t r0 = 0; r0 < G; r0 += chunk) {
        const int64_t Gc = G - r0 < chunk ? G - r0 : chunk;
        double* dg = mode >= 1 ? w.gb + Gc * M : nullptr;
        k_grid_basis<<<dim3(nblk(M, 256), (unsigned)Gc), 256, 0, s>>>(M, Gc, points + 3 * r0, w.A6,
                                                                      centers, w.Nrm, w.gb, dg);
        GSDFT_HIP(hipGetLastError());
        GSDFT_TRY(grid_orbitals(M, k, Gc, mode == 2 ? 4 : 1, Cuse, w.gb, w.pb, w, s));
        k_grid_rho<<<nblk(Gc * 64, 256), 256, 0, s>>>(Gc, k, ldk, w.pb, occ, rho + r0);
        GSDFT_HIP(hipGetLastError());
        if (mode == 1) {
            // phi (column-major M x Gc) = C (M x k) (psi occ)^T; the scaled psi goes to
            // pb + Gc ldk
            double* pocc = w.pb + Gc * ldk;
            k_grid_scale_occ<<<nblk(Gc * k, 256), 256, 0, s>>>(Gc, k, ldk, w.pb, occ, pocc);
            GSDFT_HIP(hipGetLastError());
            GSDFT_TRY(gemm_cm('T', 'N', M, Gc, k, 1.0, Cuse, ldk, pocc, ldk, 0.0, w.phi, M, s));
            k_grid_grad_phi<<<nblk(Gc * 64, 256), 256, 0, s>>>(Gc, M, w.phi, dg, grad + 3 * r0);
        } else if (mode == 2) {
            k_grid_grad_tau<<<nblk(Gc * 64, 256), 256, 0, s>>>(Gc, k, ldk, w.pb, occ,
                                                               grad + 3 * r0, tau + r0);
        }
        GSDFT_HIP(hipGetLastError());
    }
    return GSDFT_OK;
}

extern "C" int gsdft_grid_density_vjp(int64_t M, const double* quat, const double* log_scale,
                                      const double* centers, int64_t k, const double* C,
                                      const double* occ, int64_t G, const double* points,
                                      int64_t chunk, int mode, const double* v_rho,
                                      const double* v_grad, const double* v_tau, double* dquat,
                                      double* dlog_scale, double* dcenters, double* dC,
                                      void* workspace, size_t workspace_bytes, void* stream) {
    GSDFT_TRY(check_grid_args(M, k, G, chunk, mode));
    if (!quat || !log_scale || !centers || !C || !occ || !dquat || !dlog_scale || !dcenters ||
        !dC || (G > 0 && !points))
        return fail(GSDFT_ERR_ARG, "gsdft_grid_density_vjp: null argument");
    hipStream_t s = (hipStream_t)stream;
    Arena ar{(char*)workspace, workspace_bytes, 0};
    GridWs w;
    GSDFT_TRY(layout_grid(ar, M, k, chunk, mode, true, &w));
    if (!w.partial || (w.part_doubles > 0 && !w.part) || (grid_ldk(k) != k && !w.Cp))
        return fail(GSDFT_ERR_WORKSPACE, "gsdft_grid_density_vjp: workspace too small");
    const int64_t ldk = grid_ldk(k);
    const double* Cuse = nullptr;
    GSDFT_TRY(grid_c(M, k, C, w, s, &Cuse));
    const int nb = mode >= 1 ? 4 : 1;
    const int64_t slabs = (chunk + kRowsPerSlab - 1) / kRowsPerSlab;
    k_grid_fill<<<nblk(slabs * 10 * M, 256), 256, 0, s>>>(slabs * 10 * M, 0.0, w.partial);
    k_grid_fill<<<nblk(M * k, 256), 256, 0, s>>>(M * k, 0.0, dC);
    GSDFT_HIP(hipGetLastError());
    GSDFT_TRY(launch_chart(M, quat, log_scale, w.A6, w.Nrm, s));
    for (int64_t r0 = 0; r0 < G; r0 += chunk) {
        const int64_t Gc = G - r0 < chunk ? G - r0 : chunk;
        double* dg = mode >= 1 ? w.gb + Gc * M : nullptr;
        k_grid_basis<<<dim3(nblk(M, 256), (unsigned)Gc), 256, 0, s>>>(M, Gc, points + 3 * r0, w.A6,
                                                                      centers, w.Nrm, w.gb, dg);
        GSDFT_HIP(hipGetLastError());
        GSDFT_TRY(grid_orbitals(M, k, Gc, nb, Cuse, w.gb, w.pb, w, s));
        k_grid_pbar<<<nblk(Gc * k, 256), 256, 0, s>>>(Gc, k, ldk, mode, w.pb, occ,
                                                      v_rho ? v_rho + r0 : nullptr,
                                                      v_grad ? v_grad + 3 * r0 : nullptr,
                                                      v_tau ? v_tau + r0 : nullptr, w.pbar);
        GSDFT_HIP(hipGetLastError());
        // dC (column-major k x M) += pbar (k x nb Gc) [g; dg]^T (nb Gc x M)
        GSDFT_TRY(gemm_cm_split('N', 'T', k, M, nb * Gc, 1.0, w.pbar, ldk, w.gb, M, 1.0, dC, k,
                                w.part, w.part_doubles, s));
        // [gbar; dgbar] (column-major M x nb Gc) = C (M x k) pbar (k x nb Gc)
        GSDFT_TRY(gemm_cm('T', 'N', M, nb * Gc, k, 1.0, Cuse, ldk, w.pbar, ldk, 0.0, w.gbar, M,
                          s));
        const int64_t cslabs = (Gc + kRowsPerSlab - 1) / kRowsPerSlab;
        k_grid_basis_bwd<<<dim3(nblk(M, 256), (unsigned)cslabs), 256, 0, s>>>(
            M, Gc, kRowsPerSlab, points + 3 * r0, w.A6, centers, w.Nrm, w.gb, w.gbar, mode,
            w.partial);
        GSDFT_HIP(hipGetLastError());
    }
    k_grid_splat_grad<<<nblk(M, 256), 256, 0, s>>>(M, slabs, w.partial, quat, log_scale, dquat,
                                                   dlog_scale, dcenters);
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}
