// Triangular solves with the row-major lower Cholesky factor L of V + lam I:
//   L y = gamma (forward), L^T d = y (backward)  -- gs_dft/coulomb/ri.py:479's cho_solve.
//
// Single right-hand side, so the solves are HBM-bound: each reads the lower triangle once
// (N^2/2 doubles). Blocked by 128 columns, one launch per block and direction (k_trsv_fwd_step,
// k_trsv_bwd_step): the launch applies the solved block to every remaining row (forward: 16 lanes
// per row, 8 products per lane in column order, fixed 16-lane butterfly) or column (backward: one
// lane per column, row groups summed in order, group partials added in group order), and its
// workgroup 0 applies it to the neighbouring block and then solves that block: the block is staged
// in LDS and wave 0 runs the substitution (lane l holds rows l and 64 + l, each solved value is
// broadcast from its owner lane with readlane, no barrier in the 128-step chain, the diagonal
// enters as a reciprocal). The first block (forward) and the last (backward) are solved alone by
// k_trsv_diag. Every output element is updated by the same sequence of kernels in the same order,
// so results are deterministic.
#include "common.h"
#include "internal.h"

namespace gsdft {

namespace {

constexpr int kNb = 128;        // block size
constexpr int kLd = kNb + 1;    // padded LDS row

// Every kernel here runs 1024 threads per workgroup: the 128 x 128 diagonal block is staged in LDS
// (132 KB, one workgroup per CU) by all threads, 16 elements each, and solved by wave 0.
constexpr int kThreads = 1024;
constexpr int kTriLoads = kNb * kNb / kThreads;

// Strictly lower part of the diagonal block at (r0, r0), rows < nb valid, zeros elsewhere: element
// e = threadIdx.x + 1024 q is (e / 128, e % 128). Loaded into registers first so that the caller
// can issue its other loads before any of them is needed.
__device__ __forceinline__ void load_triangle(int64_t N, const double* __restrict__ L, int64_t r0,
                                              int nb, double (&v)[kTriLoads]) {
#pragma unroll
    for (int q = 0; q < kTriLoads; ++q) {
        const int e = threadIdx.x + q * kThreads;
        const int r = e >> 7, c = e & (kNb - 1);
        v[q] = (r < nb && c < r) ? L[(r0 + r) * N + r0 + c] : 0.0;
    }
}

__device__ __forceinline__ void store_triangle(const double (&v)[kTriLoads],
                                               double* __restrict__ Ls) {
#pragma unroll
    for (int q = 0; q < kTriLoads; ++q) {
        const int e = threadIdx.x + q * kThreads;
        Ls[(e >> 7) * kLd + (e & (kNb - 1))] = v[q];
    }
}

// Wave 0: substitution through the staged block. Lane l holds rows l (acc0) and 64 + l (acc1) with
// reciprocal diagonals rd0, rd1 (0 past the block's size, so those rows neither change nor
// contribute); on return acc * rd is the solution. Forward L_jj y = x; backward L_jj^T d = x.
template <bool kFwd>
__device__ __forceinline__ void solve_block(const double* __restrict__ Ls, double rd0, double rd1,
                                            double& acc0, double& acc1) {
    const int l = threadIdx.x;
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
}

// Solve the diagonal block rows [j0, j0 + nb) in place in x: forward L_jj y = x, or backward
// L_jj^T d = x.
template <bool kFwd>
__global__ __launch_bounds__(kThreads) void k_trsv_diag(int64_t N, const double* __restrict__ L,
                                                        double* __restrict__ x, int64_t j0,
                                                        int nb) {
    __shared__ double Ls[kNb * kLd];
    double v[kTriLoads];
    load_triangle(N, L, j0, nb, v);
    const int l = threadIdx.x;
    const bool h0 = l < nb, h1 = l + 64 < nb;
    double dg0 = 1.0, dg1 = 1.0, acc0 = 0.0, acc1 = 0.0;
    if (l < 64) {
        if (h0) dg0 = L[(j0 + l) * N + j0 + l], acc0 = x[j0 + l];
        if (h1) dg1 = L[(j0 + 64 + l) * N + j0 + 64 + l], acc1 = x[j0 + 64 + l];
    }
    store_triangle(v, Ls);
    __syncthreads();
    if (l >= 64) return;
    const double rd0 = h0 ? 1.0 / dg0 : 0.0, rd1 = h1 ? 1.0 / dg1 : 0.0;
    solve_block<kFwd>(Ls, rd0, rd1, acc0, acc1);
    if (h0) x[j0 + l] = acc0 * rd0;
    if (h1) x[j0 + 64 + l] = acc1 * rd1;
}

// Forward update of row i by the solved block at j0: 16 lanes per row, each holding the products of
// 8 columns (c = 2 (lane % 16) + 32 q + {0, 1}, q = 0..3, 16-byte loads, so every load instruction
// reads whole 256-byte row segments); the 8 products are added in order, then a 4-step butterfly
// over the 16 lanes. With kPair (N even, L 16-byte aligned) every pair of columns loads as one
// double2.
constexpr int kFwdLanes = 16;

// Backward update of column k by the solved block at j0: one lane per column and kBwdGroups row
// groups, each summing its rows in order; the group partials are added in group order.
constexpr int kBwdGroups = 4;
constexpr int kBwdRows = kNb / kBwdGroups;

// ------------------------------------------------------------------ fused steps
// One launch per block and direction. Workgroups 1.. apply the solved block to every row (forward)
// or column (backward) past the neighbouring block; workgroup 0 applies it to the neighbouring
// block and solves that block, so that the next launch finds it solved. Workgroup 0 issues all of
// its loads (the 128 x 128 coupling tile, the neighbouring block's triangle and diagonal, its x)
// before it uses any of them: its path is one memory round trip and the 128-step substitution,
// under the streaming of the other workgroups.

// Forward step for the solved block at j0 (full): rows i >= j1 + 128 (workgroups 1.., 128 rows
// per workgroup and iteration, two per 16-lane group) and the next block's rows [j1, j1 + nb1),
// j1 = j0 + 128 (workgroup 0, which then solves that block), take x_i -= sum_c L[i][j0 + c] y_c.
template <bool kPair>
__global__ __launch_bounds__(kThreads) void k_trsv_fwd_step(int64_t N, const double* __restrict__ L,
                                                            double* __restrict__ x, int64_t j0,
                                                            int nb1) {
    __shared__ double Ls[kNb * kLd];
    __shared__ double xs[kNb];
    const int sub = threadIdx.x & (kFwdLanes - 1);
    const int rsub = threadIdx.x >> 4;                 // 0 .. 63
    double y[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        y[2 * q] = x[j0 + 2 * sub + 32 * q];
        y[2 * q + 1] = x[j0 + 2 * sub + 32 * q + 1];
    }
    auto load_row = [&](bool live, int64_t i, double2 (&v)[4]) {
        const double* row = L + i * N + j0 + 2 * sub;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (!live) {
                v[q] = make_double2(0.0, 0.0);
            } else if constexpr (kPair) {
                v[q] = *reinterpret_cast<const double2*>(row + 32 * q);
            } else {
                v[q].x = row[32 * q];
                v[q].y = row[32 * q + 1];
            }
        }
    };
    auto dot_row = [&](const double2 (&v)[4]) {
        double p = v[0].x * y[0];
        p = __builtin_fma(v[0].y, y[1], p);
#pragma unroll
        for (int q = 1; q < 4; ++q) {
            p = __builtin_fma(v[q].x, y[2 * q], p);
            p = __builtin_fma(v[q].y, y[2 * q + 1], p);
        }
#pragma unroll
        for (int off = kFwdLanes / 2; off > 0; off >>= 1) p += __shfl_xor(p, off, kFwdLanes);
        return p;
    };
    const int64_t j1 = j0 + kNb;
    if (blockIdx.x == 0) {
        const int ra = rsub, rb = rsub + 64;
        double2 va[4], vb[4];
        load_row(ra < nb1, j1 + ra, va);
        load_row(rb < nb1, j1 + rb, vb);
        double tri[kTriLoads];
        load_triangle(N, L, j1, nb1, tri);
        double xa = 0.0, xb = 0.0;
        if (sub == 0) {
            if (ra < nb1) xa = x[j1 + ra];
            if (rb < nb1) xb = x[j1 + rb];
        }
        const int l = threadIdx.x;
        const bool h0 = l < nb1, h1 = l + 64 < nb1;
        double dg0 = 1.0, dg1 = 1.0;
        if (l < 64) {
            if (h0) dg0 = L[(j1 + l) * N + j1 + l];
            if (h1) dg1 = L[(j1 + 64 + l) * N + j1 + 64 + l];
        }
        store_triangle(tri, Ls);
        const double pa = dot_row(va), pb = dot_row(vb);
        if (sub == 0) {
            xs[ra] = ra < nb1 ? xa - pa : 0.0;
            xs[rb] = rb < nb1 ? xb - pb : 0.0;
        }
        __syncthreads();
        if (l >= 64) return;
        const double rd0 = h0 ? 1.0 / dg0 : 0.0, rd1 = h1 ? 1.0 / dg1 : 0.0;
        double acc0 = xs[l], acc1 = xs[64 + l];
        solve_block<true>(Ls, rd0, rd1, acc0, acc1);
        if (h0) x[j1 + l] = acc0 * rd0;
        if (h1) x[j1 + 64 + l] = acc1 * rd1;
        return;
    }
    for (int64_t i0 = j1 + kNb + (int64_t)(blockIdx.x - 1) * kNb; i0 < N;
         i0 += (int64_t)(gridDim.x - 1) * kNb) {
        const int64_t ia = i0 + rsub, ib = ia + 64;
        // the rows' x is read ahead of the rows and pinned after them, so that the compiler
        // keeps every load of the pass in one memory round trip rather than issuing these behind
        // the wait for the rows
        double xa = x[ia < N ? ia : N - 1], xb = x[ib < N ? ib : N - 1];
        double2 va[4], vb[4];
        load_row(ia < N, ia, va);
        load_row(ib < N, ib, vb);
        asm volatile("" : "+v"(xa), "+v"(xb));
        const double pa = dot_row(va), pb = dot_row(vb);
        if (sub == 0) {
            if (ia < N) x[ia] = xa - pa;
            if (ib < N) x[ib] = xb - pb;
        }
    }
}

// Backward step for the solved block at j0 (nb rows): columns k < jm = j0 - 128 (workgroups 1..,
// 256 columns each, 4 groups of 32 rows) and the previous block's columns [jm, j0) (workgroup 0,
// 128 columns x 8 groups of 16 rows, which then solves that block) take
// x_k -= sum_r L[j0 + r][k] d_r; each group sums its rows in order and the group partials are
// added in group order.
constexpr int kBulkCols = 256;
__global__ __launch_bounds__(kThreads) void k_trsv_bwd_step(int64_t N, const double* __restrict__ L,
                                                            double* __restrict__ x, int64_t j0,
                                                            int nb) {
    __shared__ double Ls[kNb * kLd];
    __shared__ double ds[kNb];
    __shared__ double xs[kNb];
    __shared__ double part[kThreads];
    const int t = threadIdx.x;
    const int64_t jm = j0 - kNb;
    if (blockIdx.x == 0) {
        const int c = t & (kNb - 1), g = t >> 7;       // 8 groups of 16 rows
        double col[16];
#pragma unroll
        for (int r = 0; r < 16; ++r)
            col[r] = g * 16 + r < nb ? L[(j0 + g * 16 + r) * N + jm + c] : 0.0;
        double tri[kTriLoads];
        load_triangle(N, L, jm, kNb, tri);
        double xv = 0.0, dg0 = 1.0, dg1 = 1.0;
        if (t < 64) {               // ahead of the store of d below, which waits on its load
            dg0 = L[(jm + t) * N + jm + t];
            dg1 = L[(jm + 64 + t) * N + jm + 64 + t];
        }
        if (t < kNb) {
            xv = x[jm + t];
            ds[t] = t < nb ? x[j0 + t] : 0.0;
        }
        store_triangle(tri, Ls);
        __syncthreads();
        double p = col[0] * ds[g * 16];
#pragma unroll
        for (int r = 1; r < 16; ++r) p = __builtin_fma(col[r], ds[g * 16 + r], p);
        part[g * kNb + c] = p;
        __syncthreads();
        if (t < kNb) {
            double s = part[t];
#pragma unroll
            for (int q = 1; q < kThreads / kNb; ++q) s += part[q * kNb + t];
            xs[t] = xv - s;
        }
        __syncthreads();
        if (t >= 64) return;
        const double rd0 = 1.0 / dg0, rd1 = 1.0 / dg1;
        double acc0 = xs[t], acc1 = xs[64 + t];
        solve_block<false>(Ls, rd0, rd1, acc0, acc1);
        x[jm + t] = acc0 * rd0;
        x[jm + 64 + t] = acc1 * rd1;
        return;
    }
    if (t < kNb) ds[t] = t < nb ? x[j0 + t] : 0.0;
    __syncthreads();
    const int lane = t & (kBulkCols - 1), g = t >> 8;  // 4 groups of 32 rows
    const int64_t k = (int64_t)(blockIdx.x - 1) * kBulkCols + lane;
    const bool live = k < jm;
    double acc = 0.0;
    if (live) {
        const int r0 = g * kBwdRows;
        const int r1 = r0 + kBwdRows < nb ? r0 + kBwdRows : nb;
        const double* colp = L + j0 * N + k;
#pragma unroll 8
        for (int r = r0; r < r1; ++r) acc = __builtin_fma(colp[(int64_t)r * N], ds[r], acc);
    }
    part[g * kBulkCols + lane] = acc;
    __syncthreads();
    if (g == 0 && live) {
        double s = part[lane];
#pragma unroll
        for (int q = 1; q < kBwdGroups; ++q) s += part[q * kBulkCols + lane];
        x[k] -= s;
    }
}

inline unsigned blocks_for(int64_t n, int bs) { return (unsigned)((n + bs - 1) / bs); }

}  // namespace

int launch_trsv_pair(int64_t N, const double* L, double* x, hipStream_t s) {
    const bool pair = N % 2 == 0 && reinterpret_cast<uintptr_t>(L) % 16 == 0;
    // forward: the first block alone, then one fused step per block
    k_trsv_diag<true><<<1, kThreads, 0, s>>>(N, L, x, 0, (int)(N < kNb ? N : kNb));
    for (int64_t j0 = 0; j0 + kNb < N; j0 += kNb) {
        const int nb1 = (int)((N - j0 - kNb) < kNb ? (N - j0 - kNb) : kNb);
        const int64_t rows = N - j0 - 2 * kNb;                 // bulk rows past the next block
        int64_t blocks = rows > 0 ? (rows + kNb - 1) / kNb : 0;
        if (blocks > 4096) blocks = 4096;
        if (pair)
            k_trsv_fwd_step<true><<<(unsigned)(1 + blocks), kThreads, 0, s>>>(N, L, x, j0, nb1);
        else
            k_trsv_fwd_step<false><<<(unsigned)(1 + blocks), kThreads, 0, s>>>(N, L, x, j0, nb1);
    }
    // backward: the last block alone, then one fused step per block
    const int64_t last = ((N - 1) / kNb) * kNb;
    k_trsv_diag<false><<<1, kThreads, 0, s>>>(N, L, x, last, (int)(N - last));
    for (int64_t j0 = last; j0 > 0; j0 -= kNb) {
        const int nb = (int)((N - j0) < kNb ? (N - j0) : kNb);
        const int64_t cols = j0 - kNb;                         // bulk columns before the block
        k_trsv_bwd_step<<<1 + blocks_for(cols, kBulkCols), kThreads, 0, s>>>(N, L, x, j0, nb);
    }
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}

}  // namespace gsdft
