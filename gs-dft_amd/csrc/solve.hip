// Triangular solves with the row-major lower Cholesky factor L of V + lam I:
//   L y = gamma (forward), L^T d = y (backward)  -- gs_dft/coulomb/ri.py:479's cho_solve.
//
// Single right-hand side, so the solves are HBM-bound: each reads the lower triangle once
// (N^2/2 doubles). Blocked by 128 columns. For every block one workgroup stages the block's
// strictly lower part in LDS (1024 threads, all loads in flight at once) and one wave solves it:
// lane l holds rows l and l + 64, each solved value is broadcast from its owner lane with readlane
// (no barrier in the 128-step chain), and the diagonal enters as a reciprocal. A wide kernel then
// applies the block to every remaining row (forward: 16 lanes per row, 8 products per lane in
// column order, fixed 16-lane butterfly) or column (backward: 64 columns x 4 groups of 32 rows per
// workgroup, each group in row order, the four partial sums added in group order). Every output element is updated by
// the same sequence of kernels in the same order, so results are deterministic.
#include "common.h"
#include "internal.h"

namespace gsdft {

namespace {

constexpr int kNb = 128;        // block size
constexpr int kLd = kNb + 1;    // padded LDS row

// Solve the diagonal block rows [j0, j0 + nb) in place in x: forward L_jj y = x, or backward
// L_jj^T d = x. Launched with 1024 threads: all stage the block (16 loads in flight per thread),
// wave 0 solves. The sweep always runs all 128 steps: rows and columns past nb hold zeros in LDS
// and a zero reciprocal, so they neither change nor receive anything.
constexpr int kDiagThreads = 1024;
constexpr int kDiagLoads = kNb * kNb / kDiagThreads;

template <bool kFwd>
__global__ __launch_bounds__(kDiagThreads) void k_trsv_diag(int64_t N, const double* __restrict__ L,
                                                            double* __restrict__ x, int64_t j0,
                                                            int nb) {
    __shared__ double Ls[kNb * kLd];
    double v[kDiagLoads];
#pragma unroll
    for (int q = 0; q < kDiagLoads; ++q) {
        const int e = threadIdx.x + q * kDiagThreads;
        const int r = e >> 7, c = e & (kNb - 1);
        v[q] = (r < nb && c < r) ? L[(j0 + r) * N + j0 + c] : 0.0;
    }
#pragma unroll
    for (int q = 0; q < kDiagLoads; ++q) {
        const int e = threadIdx.x + q * kDiagThreads;
        Ls[(e >> 7) * kLd + (e & (kNb - 1))] = v[q];
    }
    __syncthreads();
    if (threadIdx.x >= 64) return;
    const int l = threadIdx.x;
    const bool h0 = l < nb, h1 = l + 64 < nb;
    const double rd0 = h0 ? 1.0 / L[(j0 + l) * N + j0 + l] : 0.0;
    const double rd1 = h1 ? 1.0 / L[(j0 + 64 + l) * N + j0 + 64 + l] : 0.0;
    double acc0 = h0 ? x[j0 + l] : 0.0;
    double acc1 = h1 ? x[j0 + 64 + l] : 0.0;
    if constexpr (kFwd) {
        // rows r > c take -L[r][c] y_c; Ls is zero on and above the diagonal
#pragma unroll 16
        for (int c = 0; c < 64; ++c) {
            const double y = readlane_f64(acc0 * rd0, c);
            acc0 = __builtin_fma(-Ls[l * kLd + c], y, acc0);
            acc1 = __builtin_fma(-Ls[(64 + l) * kLd + c], y, acc1);
        }
#pragma unroll 16
        for (int c = 64; c < kNb; ++c) {
            const double y = readlane_f64(acc1 * rd1, c - 64);
            acc1 = __builtin_fma(-Ls[(64 + l) * kLd + c], y, acc1);
        }
    } else {
        // rows r < c take -L[c][r] d_c
#pragma unroll 16
        for (int c = kNb - 1; c >= 64; --c) {
            const double d = readlane_f64(acc1 * rd1, c - 64);
            acc1 = __builtin_fma(-Ls[c * kLd + 64 + l], d, acc1);
            acc0 = __builtin_fma(-Ls[c * kLd + l], d, acc0);
        }
#pragma unroll 16
        for (int c = 63; c >= 0; --c) {
            const double d = readlane_f64(acc0 * rd0, c);
            acc0 = __builtin_fma(-Ls[c * kLd + l], d, acc0);
        }
    }
    if (h0) x[j0 + l] = acc0 * rd0;
    if (h1) x[j0 + 64 + l] = acc1 * rd1;
}

constexpr int kFwdLanes = 16;                      // lanes per row in the forward update
constexpr int kFwdRowsPerGroup = 256 / kFwdLanes;   // rows per workgroup per iteration

// Forward: x_i -= sum_c L[i][j0+c] y_c for every row i >= j0 + 128 (the block is full: only the
// last block can be partial, and no row lies below it). 16 lanes per row, each holding the
// products of 8 columns (c = 2 (lane % 16) + 32 q + {0, 1}, q = 0..3, 16-byte loads, so every load
// instruction reads whole 256-byte row segments); the 8 products are added in order, then a
// 4-step butterfly over the 16 lanes.
// kPair: N even and L 16-byte aligned, so every pair of columns loads as one double2.
template <bool kPair>
__global__ __launch_bounds__(256) void k_trsv_upd_fwd(int64_t N, const double* __restrict__ L,
                                                      double* __restrict__ x, int64_t j0) {
    const int sub = threadIdx.x & (kFwdLanes - 1);
    double y[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        y[2 * q] = x[j0 + 2 * sub + 32 * q];
        y[2 * q + 1] = x[j0 + 2 * sub + 32 * q + 1];
    }
    const int64_t first = j0 + kNb;
    for (int64_t i = first + (int64_t)blockIdx.x * kFwdRowsPerGroup + (threadIdx.x >> 4); i < N;
         i += (int64_t)gridDim.x * kFwdRowsPerGroup) {
        const double* row = L + i * N + j0 + 2 * sub;
        double2 v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if constexpr (kPair) {
                v[q] = *reinterpret_cast<const double2*>(row + 32 * q);
            } else {
                v[q].x = row[32 * q];
                v[q].y = row[32 * q + 1];
            }
        }
        double p = v[0].x * y[0];
        p = __builtin_fma(v[0].y, y[1], p);
#pragma unroll
        for (int q = 1; q < 4; ++q) {
            p = __builtin_fma(v[q].x, y[2 * q], p);
            p = __builtin_fma(v[q].y, y[2 * q + 1], p);
        }
#pragma unroll
        for (int off = kFwdLanes / 2; off > 0; off >>= 1) p += __shfl_xor(p, off, kFwdLanes);
        if (sub == 0) x[i] -= p;
    }
}

constexpr int kBwdCols = 64;            // columns per workgroup of the backward update
constexpr int kBwdGroups = 4;           // row groups (one wave each)
constexpr int kBwdRows = kNb / kBwdGroups;

// Backward: x_k -= sum_r L[j0+r][k] d_r for every column k < j0. Wave g sums rows
// [g kBwdRows, (g + 1) kBwdRows) of the block for 64 consecutive columns; the four partials are
// added in group order.
__global__ __launch_bounds__(256) void k_trsv_upd_bwd(int64_t N, const double* __restrict__ L,
                                                      double* __restrict__ x, int64_t j0,
                                                      int nb) {
    __shared__ double ds[kNb];
    __shared__ double part[kBwdGroups][kBwdCols];
    if (threadIdx.x < kNb) ds[threadIdx.x] = threadIdx.x < nb ? x[j0 + threadIdx.x] : 0.0;
    __syncthreads();
    const int lane = threadIdx.x & 63, g = threadIdx.x >> 6;
    const int64_t k = blockIdx.x * (int64_t)kBwdCols + lane;
    const bool live = k < j0;
    double acc = 0.0;
    if (live) {
        const int r0 = g * kBwdRows;
        const int r1 = r0 + kBwdRows < nb ? r0 + kBwdRows : nb;
        const double* col = L + j0 * N + k;
#pragma unroll 8
        for (int r = r0; r < r1; ++r) acc = __builtin_fma(col[(int64_t)r * N], ds[r], acc);
    }
    part[g][lane] = acc;
    __syncthreads();
    if (g == 0 && live) {
        double s = part[0][lane];
#pragma unroll
        for (int q = 1; q < kBwdGroups; ++q) s += part[q][lane];
        x[k] -= s;
    }
}

inline unsigned blocks_for(int64_t n, int bs) { return (unsigned)((n + bs - 1) / bs); }

}  // namespace

int launch_trsv_pair(int64_t N, const double* L, double* x, hipStream_t s) {
    for (int64_t j0 = 0; j0 < N; j0 += kNb) {
        const int nb = (int)((N - j0) < kNb ? (N - j0) : kNb);
        k_trsv_diag<true><<<1, kDiagThreads, 0, s>>>(N, L, x, j0, nb);
        const int64_t rows = N - j0 - nb;
        if (rows > 0) {
            const int64_t blocks = (rows + kFwdRowsPerGroup - 1) / kFwdRowsPerGroup;
            const unsigned grid = (unsigned)(blocks < 8192 ? blocks : 8192);
            if (N % 2 == 0 && reinterpret_cast<uintptr_t>(L) % 16 == 0)
                k_trsv_upd_fwd<true><<<grid, 256, 0, s>>>(N, L, x, j0);
            else
                k_trsv_upd_fwd<false><<<grid, 256, 0, s>>>(N, L, x, j0);
        }
    }
    const int64_t last = ((N - 1) / kNb) * kNb;
    for (int64_t j0 = last; j0 >= 0; j0 -= kNb) {
        const int nb = (int)((N - j0) < kNb ? (N - j0) : kNb);
        k_trsv_diag<false><<<1, kDiagThreads, 0, s>>>(N, L, x, j0, nb);
        if (j0 > 0) k_trsv_upd_bwd<<<blocks_for(j0, kBwdCols), 256, 0, s>>>(N, L, x, j0, nb);
    }
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}

}  // namespace gsdft
