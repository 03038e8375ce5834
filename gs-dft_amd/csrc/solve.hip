// Triangular solves with the row-major lower Cholesky factor L of V + lam I:
//   L y = gamma (forward), L^T d = y (backward)  -- gs_dft/coulomb/ri.py:479's cho_solve.
//
// Single right-hand side, so the solves are HBM-bound: each reads the lower triangle once
// (N^2/2 doubles). Blocked by 128 columns: for every block a one-workgroup kernel solves the
// 128 x 128 diagonal block (staged in LDS, column-oriented, one barrier per column), then a wide
// kernel applies the block to every remaining row (forward: one wave per row over the row's 128
// contiguous entries, fixed butterfly) or column (backward: one lane per column, rows of the
// block in order). Every output element is updated by the same sequence of kernels in the same
// order, so results are deterministic.
#include "common.h"
#include "internal.h"

namespace gsdft {

namespace {

constexpr int kNb = 128;        // block size
constexpr int kLd = kNb + 1;    // padded LDS row

// Forward: solve the diagonal block rows [j0, j0+nb) in place in x.
__global__ __launch_bounds__(kNb) void k_trsv_diag_fwd(int64_t N, const double* __restrict__ L,
                                                       double* __restrict__ x, int64_t j0,
                                                       int nb) {
    __shared__ double Ls[kNb * kLd];
    __shared__ double ys[kNb];
    const int r = threadIdx.x;
    for (int e = r; e < nb * nb; e += kNb) {
        const int rr = e / nb, cc = e % nb;
        Ls[rr * kLd + cc] = L[(j0 + rr) * N + j0 + cc];
    }
    double acc = (r < nb) ? x[j0 + r] : 0.0;
    __syncthreads();
    for (int c = 0; c < nb; ++c) {
        if (r == c) ys[c] = acc / Ls[c * kLd + c];
        __syncthreads();
        if (r > c && r < nb) acc -= Ls[r * kLd + c] * ys[c];
    }
    if (r < nb) x[j0 + r] = ys[r];
}

// Forward: x_i -= sum_c L[i][j0+c] y_c for every row i >= j0 + nb; one wave per row.
__global__ __launch_bounds__(256) void k_trsv_upd_fwd(int64_t N, const double* __restrict__ L,
                                                      double* __restrict__ x, int64_t j0,
                                                      int nb) {
    const int lane = threadIdx.x & 63;
    const double y0 = (lane < nb) ? x[j0 + lane] : 0.0;
    const double y1 = (lane + 64 < nb) ? x[j0 + 64 + lane] : 0.0;
    const int64_t waves = (int64_t)gridDim.x * (blockDim.x >> 6);
    const int64_t first = j0 + nb;
    for (int64_t i = first + ((int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6));
         i < N; i += waves) {
        const double* row = L + i * N + j0;
        double p = (lane < nb) ? row[lane] * y0 : 0.0;
        if (lane + 64 < nb) p = __builtin_fma(row[64 + lane], y1, p);
        p = wave_sum(p);
        if (lane == 0) x[i] -= p;
    }
}

// Backward: solve L_jj^T d = x_j for the block rows [j0, j0+nb) in place.
__global__ __launch_bounds__(kNb) void k_trsv_diag_bwd(int64_t N, const double* __restrict__ L,
                                                       double* __restrict__ x, int64_t j0,
                                                       int nb) {
    __shared__ double Ls[kNb * kLd];
    __shared__ double ds[kNb];
    const int r = threadIdx.x;
    for (int e = r; e < nb * nb; e += kNb) {
        const int rr = e / nb, cc = e % nb;
        Ls[rr * kLd + cc] = L[(j0 + rr) * N + j0 + cc];
    }
    double acc = (r < nb) ? x[j0 + r] : 0.0;
    __syncthreads();
    for (int c = nb - 1; c >= 0; --c) {
        if (r == c) ds[c] = acc / Ls[c * kLd + c];
        __syncthreads();
        if (r < c) acc -= Ls[c * kLd + r] * ds[c];
    }
    if (r < nb) x[j0 + r] = ds[r];
}

// Backward: x_k -= sum_r L[j0+r][k] d_r for every column k < j0; one lane per column.
__global__ __launch_bounds__(256) void k_trsv_upd_bwd(int64_t N, const double* __restrict__ L,
                                                      double* __restrict__ x, int64_t j0,
                                                      int nb) {
    __shared__ double ds[kNb];
    if (threadIdx.x < nb) ds[threadIdx.x] = x[j0 + threadIdx.x];
    __syncthreads();
    const int64_t k = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (k >= j0) return;
    const double* col = L + j0 * N + k;
    double acc = 0.0;
    for (int r = 0; r < nb; ++r) acc = __builtin_fma(col[(int64_t)r * N], ds[r], acc);
    x[k] -= acc;
}

inline unsigned blocks_for(int64_t n, int bs) { return (unsigned)((n + bs - 1) / bs); }

}  // namespace

int launch_trsv_pair(int64_t N, const double* L, double* x, hipStream_t s) {
    for (int64_t j0 = 0; j0 < N; j0 += kNb) {
        const int nb = (int)((N - j0) < kNb ? (N - j0) : kNb);
        k_trsv_diag_fwd<<<1, kNb, 0, s>>>(N, L, x, j0, nb);
        const int64_t rows = N - j0 - nb;
        if (rows > 0) {
            const int64_t blocks = (rows + 3) / 4;
            k_trsv_upd_fwd<<<(unsigned)(blocks < 4096 ? blocks : 4096), 256, 0, s>>>(N, L, x, j0, nb);
        }
    }
    const int64_t last = ((N - 1) / kNb) * kNb;
    for (int64_t j0 = last; j0 >= 0; j0 -= kNb) {
        const int nb = (int)((N - j0) < kNb ? (N - j0) : kNb);
        k_trsv_diag_bwd<<<1, kNb, 0, s>>>(N, L, x, j0, nb);
        if (j0 > 0) k_trsv_upd_bwd<<<blocks_for(j0, 256), 256, 0, s>>>(N, L, x, j0, nb);
    }
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}

}  // namespace gsdft
