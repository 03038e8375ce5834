// Density-fitted Coulomb: product aux, metric, Cholesky, solves, and the three-centre forward
// (gamma) and reverse (J and every splat/C gradient) passes.
//
// Three-centre integral (gs_dft/coulomb/ri.py:126-151,167-185) between an isotropic aux P
// (exponent b, centre R, norm KN_P) and a pair product (precision Ah, centre Pa, KN_a):
//   (P|a) = KN_P KN_a pref sum_t w_t (prod_k Gamma_k)^(-1/2) exp(-t^2 sum_k W_k / Gamma_k)
// with Gamma_k = b L_k + t^2 (b + L_k) over the eigenvalues L_k of Ah. The kernels never
// diagonalise Ah: with a = b + t^2, c = t^2 b and s = c/a,
//   prod_k Gamma_k   = a^3 Pn(s),   Pn(s) = I3 + s (I2 + s (I1 + s)),
//   t^2 sum W/Gamma  = s Qn(s)/Pn(s), Qn(s) = I3 q0 + s ((I1 q1 - q2) + s q1),
// where I1, I2, I3 are the trace, principal-minor sum and determinant of Ah and q0 = |d|^2,
// q1 = d.Ah d, q2 = |Ah d|^2 for d = R - Pa (Cayley-Hamilton). So each node is
//   f_t = wp_t Pn^(-1/2) exp(-s Qn / Pn),   wp_t = w_t a^(-3/2),
// all positive terms, no eigh, and differentiable at degenerate Ah.
//
// Work decomposition (no atomics anywhere):
//   forward  -- one lane per pair slot; the wave walks a block's aux records (uniform node
//               tables, centre-grouped so the centre terms are shared by the exponent scales);
//               each lane keeps its partial sums per record in LDS, the block adds them in lane
//               order, and the per-block partials are summed in fixed order.
//   reverse  -- one lane per pair slot; the wave walks the aux records the same way, over slabs
//               of records small enough to stay in L2; each lane accumulates its pair's 25
//               cotangent moments per slab in registers; the slabs' moments are added in slab
//               order, and per-pair results are mapped to per-splat gradients by wave-per-splat
//               segmented sums over the CSR pair index.

#include <algorithm>
#include <cmath>
#include <mutex>
#include <type_traits>
#include <vector>

#include "common.h"
#include "internal.h"

namespace gsdft {

namespace {

constexpr int kRec = 16;      // doubles per pair record
constexpr int kAuxRec = 88;   // doubles per aux record of the reverse pass
constexpr int kAcc = 25;      // cotangent moments per pair

inline unsigned blocks_for(int64_t n, int bs) { return (unsigned)((n + bs - 1) / bs); }
// Blocks in the y or z dimension of a grid (the x dimension is bounded by its 2^32 - 1 work-items).
constexpr int64_t kMaxGridY = 65535;

// ------------------------------------------------------------------ aux

// Up to 16 exponent scales by value; longer ladders are launched in chunks (s0 = first scale of
// the chunk, so output block s0 + s holds scale sc.v[s]).
struct Scales {
    double v[16];
    int n;
    int s0;
};

// gs_dft/basis/isotropic.py:81-116, diagonal_only: the self-product of each splat.
__global__ void k_product_aux(int64_t M, const double* __restrict__ quat,
                              const double* __restrict__ log_scale,
                              const double* __restrict__ centers, Scales sc,
                              double* __restrict__ log_alpha, double* __restrict__ aux_centers) {
    const int64_t m = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (m >= M) return;
    Sym3 A, Ah;
    double N, P[3], KN;
    splat_chart(quat + 4 * m, log_scale + 3 * m, &A, &N);
    const double mu[3] = {centers[3 * m], centers[3 * m + 1], centers[3 * m + 2]};
    pair_quantities(A, A, mu, mu, N, N, &Ah, P, &KN);
    const double alpha0 = pow(det3(Ah), 1.0 / 3.0);
    for (int s = 0; s < sc.n; ++s) {
        const int64_t o = (int64_t)(sc.s0 + s) * M + m;
        log_alpha[o] = log(alpha0 * sc.v[s]);
        aux_centers[3 * o] = P[0];
        aux_centers[3 * o + 1] = P[1];
        aux_centers[3 * o + 2] = P[2];
    }
}

// gs_dft/basis/isotropic.py:106-116 with diagonal_only=False: one aux per listed pair a at its
// product centre, alpha_0 = det3(A_i + A_j)^(1/3), and the inert alpha_0 = 1 where valid[a] is 0
// (valid null: every entry live). The charts come from k_chart (A6 slots xx,yy,zz,xy,xz,yz).
__global__ void k_product_aux_pairs(int64_t n, const int32_t* __restrict__ pi,
                                    const int32_t* __restrict__ pj,
                                    const double* __restrict__ valid,
                                    const double* __restrict__ A6, const double* __restrict__ Nrm,
                                    const double* __restrict__ centers, Scales sc,
                                    double* __restrict__ log_alpha,
                                    double* __restrict__ aux_centers) {
    const int64_t a = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (a >= n) return;
    const int64_t i = pi[a], j = pj[a];
    const Sym3 Ai = load_sym(A6 + 6 * i), Aj = load_sym(A6 + 6 * j);
    const double mi[3] = {centers[3 * i], centers[3 * i + 1], centers[3 * i + 2]};
    const double mj[3] = {centers[3 * j], centers[3 * j + 1], centers[3 * j + 2]};
    Sym3 Ah;
    double P[3], KN;
    pair_quantities(Ai, Aj, mi, mj, Nrm[i], Nrm[j], &Ah, P, &KN);
    double alpha0 = pow(det3(Ah), 1.0 / 3.0);
    if (valid && valid[a] == 0.0) alpha0 = 1.0;
    for (int s = 0; s < sc.n; ++s) {
        const int64_t o = (int64_t)(sc.s0 + s) * n + a;
        log_alpha[o] = log(alpha0 * sc.v[s]);
        aux_centers[3 * o] = P[0];
        aux_centers[3 * o + 1] = P[1];
        aux_centers[3 * o + 2] = P[2];
    }
}

}  // namespace

NodeTable coulomb_table() {
    NodeTable tb{};
    for (int i = 0; i < kNodes; ++i) {
        tb.t[i] = quad_t(i);
        tb.w[i] = quad_w(i);
    }
    tb.n = kNodes;
    return tb;
}

// Gauss-Legendre on [0, omega] (gs_dft/integrals/dense.py:56-76): the roots x_i of P_12 in
// ascending order by Newton's method on the three-term recurrence, weights 2 / ((1 - x^2) P'(x)^2),
// then t = omega (x + 1) / 2 and w = omega w_x / 2.
NodeTable long_range_table(double omega) {
    NodeTable tb{};
    const int n = kLrNodes;
    for (int i = 0; i < n; ++i) {
        double x = -std::cos(kPi * (i + 0.75) / (n + 0.5));
        double dp = 1.0;
        for (int it = 0; it < 100; ++it) {
            double p0 = 1.0, p1 = x;
            for (int k = 2; k <= n; ++k) {
                const double p2 = ((2.0 * k - 1.0) * x * p1 - (k - 1.0) * p0) / k;
                p0 = p1;
                p1 = p2;
            }
            dp = n * (x * p1 - p0) / (x * x - 1.0);
            const double dx = p1 / dp;
            x -= dx;
            if (std::fabs(dx) < 1e-17) break;
        }
        double p0 = 1.0, p1 = x;
        for (int k = 2; k <= n; ++k) {
            const double p2 = ((2.0 * k - 1.0) * x * p1 - (k - 1.0) * p0) / k;
            p0 = p1;
            p1 = p2;
        }
        dp = n * (x * p1 - p0) / (x * x - 1.0);
        tb.t[i] = 0.5 * omega * (x + 1.0);
        tb.w[i] = 0.5 * omega * (2.0 / ((1.0 - x * x) * dp * dp));
    }
    tb.n = n;
    return tb;
}

namespace {

// gs_dft/basis/isotropic.py:30-39: beta = e^log_alpha, KN = (2 beta / pi)^(3/4).
__global__ void k_aux_prep(int64_t N, const double* __restrict__ log_alpha,
                           double* __restrict__ beta, double* __restrict__ kn) {
    const int64_t p = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (p >= N) return;
    const double b = exp(log_alpha[p]);
    beta[p] = b;
    kn[p] = pow(2.0 * b / kPi, 0.75);
}

__device__ __forceinline__ double boys0(double T) {
    if (T < 1e-12) return 1.0 - T / 3.0;
    return 0.5 * sqrt(kPi / T) * erf(sqrt(T));
}

// gs_dft/coulomb/ri.py:63-76 + shift_diag: F0 = boys0(rho R^2) for 1/r, or, for the long-range
// kernel erf(omega r)/r (omega > 0), sqrt(z) boys0(z rho R^2) with z = omega^2 / (omega^2 + rho).
__device__ __forceinline__ double metric_entry(double g1, double k1, double x1, double y1,
                                               double z1, double g2, double k2, double x2,
                                               double y2, double z2, double omega) {
    const double gab = g1 * g2;
    const double gsum = g1 + g2;
    const double dx = x1 - x2, dy = y1 - y2, dz = z1 - z2;
    const double PQ2 = dx * dx + dy * dy + dz * dz;
    const double rho = gab / gsum;
    const double T = rho * PQ2;
    double F0;
    if (omega != 0.0) {
        const double z = (omega * omega) / (omega * omega + rho);
        F0 = sqrt(z) * boys0(z * T);
    } else {
        F0 = boys0(T);
    }
    const double coul = kTwoPi25 / (gab * sqrt(gsum)) * F0;
    return (k1 * k2) * coul;
}

// One workgroup per 64 x 64 tile: lane l of wave w holds column q = 64 bx + l (its aux function
// read once into registers) and forms rows 64 by + w + 4 i, i < 16, whose aux data is
// wave-uniform; each row's 64 values are one contiguous 512-byte store per wave. kLower forms
// only the lower triangle (q <= p) and writes zeros above it -- tiles wholly above the diagonal
// only store zeros -- so a factorisation that follows clears only its diagonal tiles
// (k_zero_diag_tiles) instead of the whole upper triangle.
constexpr int kMetricRows = 16;
template <bool kLower>
__global__ __launch_bounds__(256) void k_metric(int64_t N, const double* __restrict__ beta,
                                                const double* __restrict__ kn,
                                                const double* __restrict__ R, double lam,
                                                double omega, double* __restrict__ V) {
    const int64_t q = (int64_t)blockIdx.x * 64 + (threadIdx.x & 63);
    const int64_t p0 = (int64_t)blockIdx.y * (4 * kMetricRows) + (threadIdx.x >> 6);
    if (q >= N) return;
    if (kLower && (int64_t)blockIdx.x * 64 > (int64_t)blockIdx.y * (4 * kMetricRows) +
                                                 4 * kMetricRows - 1) {     // workgroup-uniform
#pragma unroll 4
        for (int i = 0; i < kMetricRows; ++i) {
            const int64_t p = p0 + 4 * i;
            if (p < N) V[p * N + q] = 0.0;
        }
        return;
    }
    const double g2 = beta[q], k2 = kn[q], x2 = R[3 * q], y2 = R[3 * q + 1], z2 = R[3 * q + 2];
    for (int i = 0; i < kMetricRows; ++i) {
        const int64_t p = p0 + 4 * i;                                      // wave-uniform
        if (p >= N) break;
        if (kLower && q > p) {
            V[p * N + q] = 0.0;
            continue;
        }
        double v = metric_entry(beta[p], kn[p], R[3 * p], R[3 * p + 1], R[3 * p + 2], g2, k2, x2,
                                y2, z2, omega);
        if (p == q) v += lam;
        V[p * N + q] = v;
    }
}

__global__ void k_fill(int64_t n, double v, double* __restrict__ out) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i < n) out[i] = v;
}

__global__ void k_zero_upper(int64_t N, double* __restrict__ V) {
    const int64_t q = blockIdx.x * 64 + (threadIdx.x & 63);
    const int64_t p = blockIdx.y * 4 + (threadIdx.x >> 6);
    if (p >= N || q >= N || q <= p) return;
    V[p * N + q] = 0.0;
}

// scale * a.b in one block, fixed summation order.
__global__ __launch_bounds__(1024) void k_scaled_dot(int64_t N, const double* __restrict__ a,
                                                     const double* __restrict__ b, double scale,
                                                     double* __restrict__ out) {
    __shared__ double part[1024];
    double s = 0.0;
    for (int64_t i = threadIdx.x; i < N; i += 1024) s += a[i] * b[i];
    part[threadIdx.x] = s;
    __syncthreads();
    for (int w = 512; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) part[threadIdx.x] += part[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) *out = scale * part[0];
}

// The same as two fixed-order stages for long vectors: block b of the first stage sums the
// elements [b kDotChunk, (b + 1) kDotChunk) (thread-strided, then a tree), the second adds the
// block sums. The partition does not depend on N, so appended zero entries change nothing.
constexpr int64_t kDotChunk = 8192;
inline int64_t dot_blocks(int64_t N) { return std::max<int64_t>(1, (N + kDotChunk - 1) / kDotChunk); }

__global__ __launch_bounds__(256) void k_dot_part(int64_t N, int64_t chunk,
                                                  const double* __restrict__ a,
                                                  const double* __restrict__ b,
                                                  double* __restrict__ part) {
    __shared__ double red[256];
    const int64_t i0 = blockIdx.x * chunk, i1 = min(N, i0 + chunk);
    double s = 0.0;
    for (int64_t i = i0 + threadIdx.x; i < i1; i += 256) s = __builtin_fma(a[i], b[i], s);
    red[threadIdx.x] = s;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) part[blockIdx.x] = red[0];
}

__global__ __launch_bounds__(256) void k_dot_finish(int64_t blocks, const double* __restrict__ part,
                                                    double scale, double* __restrict__ out) {
    __shared__ double red[256];
    double s = 0.0;
    for (int64_t i = threadIdx.x; i < blocks; i += 256) s += part[i];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
        __syncthreads();
    }
    if (threadIdx.x == 0) *out = scale * red[0];
}

// scale * a.b into *out (device), with part holding dot_blocks(N) doubles of scratch.
int launch_scaled_dot(int64_t N, const double* a, const double* b, double scale, double* out,
                      double* part, hipStream_t s) {
    const int64_t blocks = dot_blocks(N);
    k_dot_part<<<(unsigned)blocks, 256, 0, s>>>(N, kDotChunk, a, b, part);
    k_dot_finish<<<1, 256, 0, s>>>(blocks, part, scale, out);
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}

// ------------------------------------------------------------------ pair records

// Workgroups are dispatched to the 8 XCDs in turn (workgroup b to XCD b mod 8). A launch of
// xcd_grid(nb) workgroups in which workgroup b takes logical block xcd_block(nb) = (b mod 8) chunk
// + b / 8 (chunk = ceil(nb / 8); -1 past nb) gives each XCD one contiguous range of the nb logical
// blocks, so neighbouring blocks' reads of shared rows meet in that XCD's L2.
inline unsigned xcd_grid(int64_t nb) { return (unsigned)(8 * ((nb + 7) / 8)); }

__device__ __forceinline__ int64_t xcd_block(int64_t nb) {
    const int64_t chunk = (nb + 7) / 8;
    const int64_t lb = (int64_t)(blockIdx.x % 8) * chunk + blockIdx.x / 8;
    return lb < nb ? lb : -1;
}

// q_a = w_a sum_o occ_o C_io C_jo (gs_dft/coulomb/ri.py:456; w_a = 1 for a null weight); G lanes
// per pair, the grid striding over the pairs (G n work-items can pass a grid dimension's 2^32 - 1).
template <int G>
__global__ __launch_bounds__(256) void k_pair_density(int64_t n, const int32_t* __restrict__ pi,
                                                      const int32_t* __restrict__ pj,
                                                      const double* __restrict__ weight, int64_t k,
                                                      const double* __restrict__ C,
                                                      const double* __restrict__ occ,
                                                      double* __restrict__ q) {
    const int l = threadIdx.x % G;
    const int64_t stride = (int64_t)gridDim.x * (blockDim.x / G);
    // the G lanes of a pair share a, so a group is wholly in or out of the loop and the butterfly
    // (lane offsets below G) reads only lanes of its own group
    for (int64_t a = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) / G; a < n; a += stride) {
        const int64_t i = pi[a], j = pj[a];
        double s = 0.0;
        for (int64_t o = l; o < k; o += G) s += (occ[o] * C[i * k + o]) * C[j * k + o];
        for (int off = G / 2; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
        if (l == 0) q[a] = (weight ? weight[a] : 1.0) * s;
    }
}

// The same for 64 lanes per pair (k > 32), one wave per run of kRun consecutive pairs: the lane's
// occ_o C_io (o = lane + 64 t, kR values per lane, k <= 64 kR) stay in registers while i does not
// change -- on a list sorted by i, for most of a splat's partners -- so a pair reads only C_j from
// the cache hierarchy instead of C_i, C_j and occ. Each product and each lane's sum are formed in
// the order of k_pair_density<64>, so q is bit-identical.
constexpr int64_t kDensityRun = 16;
template <int kR>
__global__ __launch_bounds__(256) void k_pair_density_run(int64_t n,
                                                          const int32_t* __restrict__ pi,
                                                          const int32_t* __restrict__ pj,
                                                          const double* __restrict__ weight,
                                                          int64_t k,
                                                          const double* __restrict__ C,
                                                          const double* __restrict__ occ,
                                                          double* __restrict__ q) {
    const int lane = threadIdx.x & 63;
    const int64_t a0 = ((blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6) * kDensityRun;
    const int64_t a1 = min(n, a0 + kDensityRun);
    double ci[kR];
    int64_t cur = -1;
    for (int64_t a = a0; a < a1; ++a) {                  // wave-uniform
        const int64_t i = pi[a], j = pj[a];
        // every load of a row is issued before any is used (addresses clamped in range; the
        // values past k are never added), so a row costs one memory round trip
        if (i != cur) {                                  // wave-uniform
            double cv[kR], ov[kR];
#pragma unroll
            for (int t = 0; t < kR; ++t) {
                const int64_t o = min((int64_t)(lane + 64 * t), k - 1);
                cv[t] = C[i * k + o];
                ov[t] = occ[o];
            }
#pragma unroll
            for (int t = 0; t < kR; ++t) ci[t] = ov[t] * cv[t];
            cur = i;
        }
        double cj[kR];
#pragma unroll
        for (int t = 0; t < kR; ++t) cj[t] = C[j * k + min((int64_t)(lane + 64 * t), k - 1)];
        double s = 0.0;
#pragma unroll
        for (int t = 0; t < kR; ++t)
            if (lane + 64 * t < k) s += ci[t] * cj[t];
        for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
        if (lane == 0) q[a] = (weight ? weight[a] : 1.0) * s;
    }
}

// Pair record: I1 I2 I3 | Ah (6) | Pa (3) | coef = KN q pref | KN | q | pad.
__global__ void k_pair_rec(int64_t n, const int32_t* __restrict__ pi,
                           const int32_t* __restrict__ pj, const double* __restrict__ A6,
                           const double* __restrict__ mu, const double* __restrict__ Nrm,
                           const double* __restrict__ q, double* __restrict__ rec) {
    const int64_t a = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (a >= n) return;
    const int64_t i = pi[a], j = pj[a];
    const Sym3 Ai = load_sym(A6 + 6 * i), Aj = load_sym(A6 + 6 * j);
    const double mui[3] = {mu[3 * i], mu[3 * i + 1], mu[3 * i + 2]};
    const double muj[3] = {mu[3 * j], mu[3 * j + 1], mu[3 * j + 2]};
    Sym3 Ah;
    double P[3], KN;
    pair_quantities(Ai, Aj, mui, muj, Nrm[i], Nrm[j], &Ah, P, &KN);
    double* r = rec + kRec * a;
    r[0] = Ah.xx + Ah.yy + Ah.zz;
    r[1] = Ah.xx * Ah.yy + Ah.xx * Ah.zz + Ah.yy * Ah.zz - Ah.xy * Ah.xy - Ah.xz * Ah.xz
         - Ah.yz * Ah.yz;
    r[2] = det3(Ah);
    r[3] = Ah.xx; r[4] = Ah.yy; r[5] = Ah.zz; r[6] = Ah.xy; r[7] = Ah.xz; r[8] = Ah.yz;
    r[9] = P[0]; r[10] = P[1]; r[11] = P[2];
    r[12] = KN * kPref3c * q[a];
    r[13] = KN;
    r[14] = q[a];
    r[15] = 0.0;
}

// Node constants of one aux exponent b for the first tb.n nodes of the table:
// s_t = t^2 b / (b + t^2), wp_t = w_t (b + t^2)^(-3/2).
__device__ __forceinline__ void node_consts(double b, const NodeTable& tb, double s[kNodes],
                                            double wp[kNodes]) {
#pragma unroll
    for (int t = 0; t < kNodes; ++t) {
        if (t >= tb.n) break;
        const double t2 = tb.t[t] * tb.t[t];
        const double a = b + t2;
        s[t] = t2 * b / a;
        wp[t] = tb.w[t] / (a * sqrt(a));
    }
}

// ------------------------------------------------------------------ node screen
// The nodes run in increasing t, and the exponent of node t is
//   z_t = s_t Qn/Pn = sum_k dp_k^2 / (1/s_t + 1/L_k),   1/s_t = 1/t^2 + 1/b,
// (dp = d in the eigenbasis of Ah, L_k its eigenvalues), which grows with t. Once z_t > kSkipZ on
// every live lane of a wave, each remaining node is below e^-36 ~ 2.3e-16 of its own prefactor
// wp_t Pn^(-1/2), and the prefactors sum to the integral at zero separation, so the wave leaves
// the node loop. The reverse pass screens the same way; its node terms carry e^-z times z^m s^k
// (m <= 1, k <= 3), and z e^-z <= 36 e^-36 ~ 8e-15 beyond the cut. Measured on sampled (P|a) of
// the 700-atom globule (M = 20000) and the C20H42 chain against all 20 nodes: every integral is
// bit-identical in double precision, and the z-weighted reverse terms move by <= 1.2e-15
// relative. Checks follow every node from kFirstSkip on, before which z_t <= t^2 |d|^2 stays
// small for any pair within ~30 Bohr.
constexpr double kSkipZ = 36.0;
constexpr int kFirstSkip = 5;

template <int kN = kNodes>
__host__ __device__ constexpr bool screen_after(int t) {
    return t >= kFirstSkip && t + 1 < kN;
}

// Lanes past the end of the work hold a centre kFarAway Bohr off (z ~ 1e40 at every node from
// kFirstSkip on), so they never keep a wave in the loop and need no mask of their own.
constexpr double kFarAway = 1e20;

// True once every lane of the wave has z > kSkipZ, tested on zh = z - 1/2 (node_val_h) or on the
// forward's arg = zh - eps/2 (node_arg_h), which differs from zh by less than 6e-8.
__device__ __forceinline__ bool wave_all_beyond_h(double zh) {
    return __builtin_amdgcn_ballot_w64(!(zh > kSkipZ - 0.5)) == 0;
}

// The record's "first" flag (1.0 or 0.0): tested on its bits, so the wave-uniform test is a scalar
// compare rather than a vector one.
__device__ __forceinline__ bool new_centre(const double* __restrict__ x) {
    return __builtin_bit_cast(uint64_t, x[5]) != 0;
}

// Node constants of one aux record (layout below): s_t, wh_t = wp_t s_t^(-1/2) e^(-1/2) / K, s_t^2
// and 1/s_t, for the scaled node form (node_val_h) and exp_neg_tab_k of the three-centre passes;
// `scale` multiplies the weight (the record's u, for the reverse pass that folds it in). Stored
// node-major from offset 8 (node t at 8 + 4 t): the four values a node reads are one 32-byte run,
// a single scalar load, and two nodes share a cache line.
constexpr double kExpMinusHalf = 0x1.368b2fc6f960ap-1;     // e^(-1/2), correctly rounded

__host__ __device__ constexpr int rec_s(int t) { return 8 + 4 * t; }
__host__ __device__ constexpr int rec_wh(int t) { return 8 + 4 * t + 1; }
__host__ __device__ constexpr int rec_s2(int t) { return 8 + 4 * t + 2; }
__host__ __device__ constexpr int rec_is(int t) { return 8 + 4 * t + 3; }

__device__ __forceinline__ void put_node_consts(double* o, int t, double s, double wp,
                                                double scale = 1.0) {
    o[rec_s(t)] = s;
    o[rec_wh(t)] = wp / sqrt(s) * (kExpMinusHalf / kExpPolyK) * scale;
    o[rec_s2(t)] = s * s;
    o[rec_is(t)] = 1.0 / s;
}

// The forward's records (k_gamma_fwd_pairs) hold the weight split for exp_neg_tab_k_w in the
// same four slots: s_t, -ln w'_t, S_t, 1/s_t with wh_t = 2^n w'_t (fold_weight).
__host__ __device__ constexpr int rec_lw(int t) { return 8 + 4 * t + 1; }
__host__ __device__ constexpr int rec_S(int t) { return 8 + 4 * t + 2; }

__device__ __forceinline__ void put_fwd_node_consts(double* o, int t, double s, double wp) {
    double S;
    o[rec_s(t)] = s;
    o[rec_lw(t)] = fold_weight(wp / sqrt(s) * (kExpMinusHalf / kExpPolyK), &S);
    o[rec_S(t)] = S;
    o[rec_is(t)] = 1.0 / s;
}

// body(std::integral_constant<int, t>) for t = 0, 1, ..., kN - 1 until it returns true: a fully
// unrolled node loop with early exits (node tables stay in registers). Returns the number of
// nodes evaluated (wave-uniform).
template <int T, int kN = kNodes, class Body>
__device__ __forceinline__ uint32_t node_loop(Body& body) {
    if constexpr (T < kN) {
        if (body(std::integral_constant<int, T>{})) return T + 1;
        return node_loop<T + 1, kN>(body);
    } else {
        return kN;
    }
}

// Profiling only: adds this wave's node evaluations over its live lanes to *work.
__device__ __forceinline__ void count_work(unsigned long long* work, bool live, uint32_t nodes) {
    if (!work) return;
    const uint64_t lanes = __builtin_popcountll(__builtin_amdgcn_ballot_w64(live));
    if ((threadIdx.x & 63) == 0) atomicAdd(work, (unsigned long long)(lanes * nodes));
}

// ------------------------------------------------------------------ forward

// Forward with one lane per pair slot (the reverse's slot order) and the aux records of the reverse
// (centre-grouped, wave-uniform): block (s, g) of the 2-D grid (ceil(N / kFwdRecs), pair groups)
// sums the pair slots [g kFwdPairs, (g + 1) kFwdPairs) against the kFwdRecs aux slots from
// s kFwdRecs on. The record blocks (x) run fastest, so the workgroups dispatched together share
// their pair slots (read once into L2) and differ only in their aux records. (One dimension of a
// grid holds at most 2^32 - 1 work-items: a 1-D grid of both would pass that at 20 M pairs.) The centre-dependent terms (d, Ah d, q0..q2)
// are formed once per centre and shared by its exponent scales, and the wave's node screen acts on
// 64 pairs in precision band + Morton order. Each lane keeps its running sums of coef_a F(P, a) for
// the block's records in LDS; at the end the 256 lane sums of each record are added in lane order
// and scaled by KN_P (the record's u): partial[g * N + slot]. Twelve records per block keep the
// LDS at 26 KB, so six workgroups (six waves per SIMD, within the kernel's 60 registers) share a
// CU; 16 records (34 KB, four waves per SIMD) were 1.9% slower and 8 or 10 records 0.9% and 1.6%.
// The sums do not depend on the block size: each lane adds its pairs to a record's sum in the
// same order, and the lanes are added in lane order.
constexpr int kFwdRecs = 12;
constexpr int64_t kFwdPairs = 8192;

__global__ __launch_bounds__(256) void k_gamma_fwd_pairs(int64_t n,
                                                         const double* __restrict__ rec,
                                                         int64_t N,
                                                         const double* __restrict__ aux,
                                                         double* __restrict__ partial,
                                                         unsigned long long* __restrict__ work) {
    __shared__ double tab[256];
    __shared__ double acc[kFwdRecs][256];
    for (int i = threadIdx.x; i < 256; i += blockDim.x) tab[i] = exp2_frac_lead(i);
#pragma unroll
    for (int j = 0; j < kFwdRecs; ++j) acc[j][threadIdx.x] = 0.0;
    __syncthreads();
    const int64_t q0 = (int64_t)blockIdx.x * kFwdRecs, g = blockIdx.y;
    const int nrec = (int)min((int64_t)kFwdRecs, N - q0);
    const int64_t a_begin = g * kFwdPairs;
    const int64_t a_end = min(n, a_begin + kFwdPairs);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const double c256 = vgpr_const(kNegC256);
    uint64_t lane_nodes = 0;                 // profiling: node evaluations over live lanes
    for (int64_t a0 = a_begin + 64 * wave; a0 < a_end; a0 += 256) {      // wave-uniform
        const int64_t a = a0 + lane;
        const bool live = a < a_end;
        const uint64_t lanes = __builtin_popcountll(__builtin_amdgcn_ballot_w64(live));
        const double* __restrict__ r = rec + kRec * (live ? a : a0);
        const double I1 = r[0], I2 = r[1], I3 = r[2];
        const double xx = r[3], yy = r[4], zz = r[5], xy = r[6], xz = r[7], yz = r[8];
        const double Px = live ? r[9] : kFarAway, Py = live ? r[10] : kFarAway,
                     Pz = live ? r[11] : kFarAway;
        const double coef = live ? r[12] : 0.0;
        double q0d = 0, q1 = 0, X0 = 0, rr = 0, cf = coef;
        // Each record's centre, new-centre flag and node-0 constants are read one record ahead
        // (the first record's here), so their scalar loads overlap a node loop instead of
        // stalling the record's start.
        const double* __restrict__ xf = aux + kAuxRec * q0;
        double c_x = xf[0], c_y = xf[1], c_z = xf[2];
        double c_s = xf[rec_s(0)], c_lw = xf[rec_lw(0)], c_S = xf[rec_S(0)],
               c_is = xf[rec_is(0)];
        uint64_t c_new = 1;                          // the flag's bits, tested when used
        for (int j = 0; j < nrec; ++j) {
            const double* __restrict__ x = aux + kAuxRec * (q0 + j);
            const double Rx = c_x, Ry = c_y, Rz = c_z;
            double n_s = c_s, n_lw = c_lw, n_S = c_S, n_is = c_is;
            const bool fresh = c_new != 0;
            if (j + 1 < nrec) {                      // wave-uniform
                const double* __restrict__ xn = x + kAuxRec;
                c_x = xn[0]; c_y = xn[1]; c_z = xn[2];
                c_s = xn[rec_s(0)]; c_lw = xn[rec_lw(0)]; c_S = xn[rec_S(0)];
                c_is = xn[rec_is(0)];
                c_new = __builtin_bit_cast(uint64_t, xn[5]);
            }
            if (fresh) {                             // wave-uniform
                const double dx = Rx - Px, dy = Ry - Py, dz = Rz - Pz;
                const double ax = __builtin_fma(xx, dx, __builtin_fma(xy, dy, xz * dz));
                const double ay = __builtin_fma(xy, dx, __builtin_fma(yy, dy, yz * dz));
                const double az = __builtin_fma(xz, dx, __builtin_fma(yz, dy, zz * dz));
                q0d = __builtin_fma(dx, dx, __builtin_fma(dy, dy, dz * dz));
                q1 = __builtin_fma(dx, ax, __builtin_fma(dy, ay, dz * az));
                const double q2 = __builtin_fma(ax, ax, __builtin_fma(ay, ay, az * az));
                X0 = I3 * q0d;
                rr = __builtin_fma(I1, q1, -q2);
                cf = (q0d == q0d) ? coef : q0d;      // a NaN centre propagates
            }
            double F = 0.0;
            // each node's constants are read one node ahead, so their scalar load overlaps the
            // previous node's arithmetic
            // The node weight rides in the exponent (exp_neg_tab_k_w): with y0 ~ Pr^(-1/2),
            // h = y0^2 and 1 + eps = 2 - Pr h, the term is y0 e^-(a (1 + eps) - ln w') 2^n for
            // a = Qn h - 1/2 (node_arg_h's argument, formed as one fma with ln w'), so no
            // multiply by the weight is left. The screen tests a, which differs from
            // a (1 + eps) by less than 4e-6 where it matters.
            auto node = [&](auto tc) {
                constexpr int t = decltype(tc)::value;
                const double st = n_s, lw = n_lw, S = n_S, is = n_is;
                if constexpr (t + 1 < kNodes) {
                    n_s = x[rec_s(t + 1)];
                    n_lw = x[rec_lw(t + 1)];
                    n_S = x[rec_S(t + 1)];
                    n_is = x[rec_is(t + 1)];
                }
                const double Pr = __builtin_fma(is, I3, __builtin_fma(st, I1 + st, I2));
                const double Qn = __builtin_fma(st, __builtin_fma(st, q1, rr), X0);
                const double y0 = __builtin_amdgcn_rsq(Pr);
                const double h = y0 * y0;
                const double e1 = __builtin_fma(-Pr, h, 2.0);
                const double a = __builtin_fma(Qn, h, -0.5);
                F = __builtin_fma(y0, exp_neg_tab_k_w(__builtin_fma(a, e1, lw), S, c256, tab), F);
                // keep the next node's loads ahead of the early exit (not sunk past it)
                if constexpr (t + 1 < kNodes)
                    asm volatile("" ::"s"(n_s), "s"(n_lw), "s"(n_S), "s"(n_is));
                return screen_after(t) && wave_all_beyond_h(a);
            };
            lane_nodes += lanes * node_loop<0>(node);
            acc[j][threadIdx.x] = __builtin_fma(F, cf, acc[j][threadIdx.x]);
        }
    }
    if (work && (threadIdx.x & 63) == 0) atomicAdd(work, (unsigned long long)lane_nodes);
    __syncthreads();
    if ((int)threadIdx.x < nrec) {
        double sum = 0.0;
        for (int l = 0; l < 256; ++l) sum += acc[threadIdx.x][l];
        partial[g * N + q0 + threadIdx.x] =
            sum * aux[kAuxRec * (q0 + threadIdx.x) + 3];
    }
}

// gamma[p] = sum over pair groups of partial[g * N + slot(p)], in group order.
__global__ void k_slot_sum(int64_t N, int64_t G, int64_t groups, const double* __restrict__ partial,
                           double* __restrict__ gamma) {
    const int64_t p = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (p >= N) return;
    const int64_t q = aux_slot(p, N, G);
    double s = 0.0;
    for (int64_t g = 0; g < groups; ++g) s += partial[g * N + q];
    gamma[p] = s;
}

// ------------------------------------------------------------------ reverse

// Cross-lane moves of doubles (two 32-bit halves each). swap32(x, y): x' = [x lanes 0-31, y lanes
// 0-31], y' = [x lanes 32-63, y lanes 32-63]; swap16 does the same with the 16-lane rows of each
// half (v_permlane32_swap / v_permlane16_swap); dpp<ctrl> reads the lane that a DPP control names
// (0x140 row mirror: lane 15 - i of the row; 0x141 half-row mirror: 7 - i of the 8; 0x4e, 0xb1:
// lane i ^ 2, i ^ 1).
__device__ __forceinline__ void swap32(double& x, double& y) {
    const uint64_t a = __builtin_bit_cast(uint64_t, x), b = __builtin_bit_cast(uint64_t, y);
    const auto lo = __builtin_amdgcn_permlane32_swap((uint32_t)a, (uint32_t)b, false, false);
    const auto hi = __builtin_amdgcn_permlane32_swap((uint32_t)(a >> 32), (uint32_t)(b >> 32),
                                                     false, false);
    x = __builtin_bit_cast(double, ((uint64_t)hi[0] << 32) | lo[0]);
    y = __builtin_bit_cast(double, ((uint64_t)hi[1] << 32) | lo[1]);
}

__device__ __forceinline__ void swap16(double& x, double& y) {
    const uint64_t a = __builtin_bit_cast(uint64_t, x), b = __builtin_bit_cast(uint64_t, y);
    const auto lo = __builtin_amdgcn_permlane16_swap((uint32_t)a, (uint32_t)b, false, false);
    const auto hi = __builtin_amdgcn_permlane16_swap((uint32_t)(a >> 32), (uint32_t)(b >> 32),
                                                     false, false);
    x = __builtin_bit_cast(double, ((uint64_t)hi[0] << 32) | lo[0]);
    y = __builtin_bit_cast(double, ((uint64_t)hi[1] << 32) | lo[1]);
}

template <int kCtrl>
__device__ __forceinline__ double dpp(double v) {
    const uint64_t a = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)a, kCtrl, 0xf, 0xf,
                                                              false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(a >> 32), kCtrl,
                                                              0xf, 0xf, false);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Sums of three values over the 64 lanes of a wave (v0, v1 paired across lane bit 5, v2 with a
// zero; then across bit 4; then the row steps of wave_sum_x): the totals of v0, v2 and v1 end in
// lanes 0, 16 and 32. Returns this lane's total and sets *comp to its component there, -1
// elsewhere. Fixed order.
__device__ __forceinline__ double wave_sum3(const double v[3], int* comp) {
    double x = v[0], y = v[1];
    swap32(x, y);
    double u0 = x + y;
    x = v[2]; y = 0.0;
    swap32(x, y);
    double u1 = x + y;
    swap16(u0, u1);
    double w = u0 + u1;
    w += dpp<0x140>(w);
    w += dpp<0x141>(w);
    w += dpp<0x4e>(w);
    w += dpp<0xb1>(w);
    const int L = threadIdx.x & 63;
    *comp = L == 0 ? 0 : L == 32 ? 1 : L == 16 ? 2 : -1;
    return w;
}


// Aux record: R (3) | u = dgamma_P * scale * KN_P | b | first | pad (2) | per node t: s_t, wh_t,
// s_t^2, 1/s_t (put_node_consts; with fold == kAuxFoldU the weights carry u; with
// fold == kAuxForward the forward's split weights instead, put_fwd_node_consts). Records are stored
// centre-grouped: with G = N / M exponent scales (the product aux is scale-major, P = s M + m,
// every scale of splat m at one centre), the record of P sits at slot m G + s, so the scales
// sharing a centre are consecutive; otherwise (N not a multiple of M) in aux order. "first" is 1
// where the centre differs bitwise from the previous slot's (or at slot 0): the reverse kernel
// recomputes the centre-dependent terms only there, whatever the aux holds.
// (aux_slot / aux_of_slot: common.h)

enum AuxFold { kAuxPlain = 0, kAuxFoldU = 1, kAuxForward = 2 };

__global__ void k_aux_bwd_prep(int64_t N, int64_t G, const double* __restrict__ beta,
                               const double* __restrict__ kn, const double* __restrict__ R,
                               const double* __restrict__ dgamma,
                               const double* __restrict__ dscale, int fold, NodeTable tb,
                               double* __restrict__ out) {
    const int64_t p = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (p >= N) return;
    const double b = beta[p];
    double s[kNodes], wp[kNodes];
    node_consts(b, tb, s, wp);
    const int64_t slot = aux_slot(p, N, G);
    double* o = out + kAuxRec * slot;
    o[0] = R[3 * p]; o[1] = R[3 * p + 1]; o[2] = R[3 * p + 2];
    const double u = (dgamma ? dgamma[p] : 1.0) * (dscale ? *dscale : 1.0) * kn[p];
    o[3] = u;
    bool first = true;
    if (slot > 0) {
        const int64_t q = aux_of_slot(slot - 1, N, G);
        first = !(__builtin_bit_cast(uint64_t, R[3 * q]) == __builtin_bit_cast(uint64_t, R[3 * p]) &&
                  __builtin_bit_cast(uint64_t, R[3 * q + 1]) ==
                      __builtin_bit_cast(uint64_t, R[3 * p + 1]) &&
                  __builtin_bit_cast(uint64_t, R[3 * q + 2]) ==
                      __builtin_bit_cast(uint64_t, R[3 * p + 2]));
    }
    o[4] = b; o[5] = first ? 1.0 : 0.0; o[6] = 0.0; o[7] = 0.0;
    for (int t = 0; t < kNodes; ++t) {
        if (t < tb.n && fold == kAuxForward) {
            put_fwd_node_consts(o, t, s[t], wp[t]);
        } else if (t < tb.n) {
            put_node_consts(o, t, s[t], wp[t], fold == kAuxFoldU ? u : 1.0);
        } else {            // slots past the table: never read by a kernel of tb.n nodes
            o[rec_s(t)] = 0.0;
            o[rec_wh(t)] = 0.0;
            o[rec_s2(t)] = 0.0;
            o[rec_is(t)] = 0.0;
        }
    }
}

// One lane per pair slot; accumulates over a slab of aux records (u = dgamma_P KN_P)
//   jt = sum u F,  T1/T2/T3 = sum u dF/dI1,I2,I3 (through Pn and Qn),
//   Vc = sum u dQ0 d, Va = sum u dQ1 d, Vb = sum u dQ2 d, Sa = sum u dQ1 d d^T, Sb = sum u dQ2 d d^T
// where dQk = sum_t (df/dQn) s^k = -sum_t g_t s^(k+1), dPk = sum_t (df/dPn) s^k, with
// f_t = wp_t y e^-z, y = Pn^(-1/2), z = s Qn / Pn, g_t = f_t / Pn and df/dPn = g_t (z - 1/2).
// Records sharing a centre are consecutive, so d = R - Pa and the d-moments are formed once per
// centre: C0..C2 = sum u dQ0..2 over the group, then Vc += C0 d, ..., Sb += C2 d d^T.
// Each node runs in the scaled form Pr = Pn/s (node_val_h): G = f/Pr = g s, so the node sums are
// gs1..3 = sum G (1, s, s^2) = sum g s^(1..3) and dP0..2 = sum G (z - 1/2) (1/s, 1, s).
// With kFold the record weights already carry u (k_aux_bwd_prep with fold): the node sums then run
// over all records of a centre and are turned into jt, T1..T3 and C0..C2 once per centre (flush),
// since every per-record term is linear in u and q0, q1 are the centre's.
// With kLaneU the cotangent of (P|a) is not separable: lane slot a holds the group g = uperm[a] of
// list entries sharing one product Gaussian, and u = x[3] * sum over e in [uptr[g], uptr[g + 1])
// of ut[e * ldu + p] (the exchange's dE/d(P|a) per entry, rows in key order), added in order; with
// ugroup the group's entries share one cotangent row, ut[g * ldu + p], and u = x[3] * (that row
// times the entry count uptr[g + 1] - uptr[g]).
// With kAtomF the records are nuclei (point charges) and the pass also forms every nucleus' force
// from the same node sums: per (nucleus p, pair a) the vector 2 KN_a q_a (f0 d + f1 Ah d + f2 Ah^2 d),
// f0 = -I3 sum g s, f1 = -(I1 sum g s^2 + sum g s^3), f2 = sum g s^2 (dF/dR of
// gs_dft/ks/forces.py:53-77 through pairs.py:348-370), summed over the wave (wave_sum3), then over
// the four waves in LDS per chunk of 64 nuclei, into atom_part[pair block][p][3] (times -Z_p 2 pi
// later).
constexpr int kAtomChunk = 64;

// The nuclear-force form (kAtomF) is held to four waves per SIMD (128 registers, a 20-byte spill
// outside the node loop): 1.6% faster than the three its 134 registers allowed. The other forms
// keep their allocation (for kLaneU four waves cost a 32-byte spill and 2.6%).
template <bool kLaneU, bool kAtomF = false, bool kFold = false, int kN = kNodes>
__global__ __launch_bounds__(256, kAtomF ? 4 : 1) void k_gamma_bwd(
    int64_t n, const double* __restrict__ rec, int64_t N, const double* __restrict__ aux,
    int64_t per_slab, double* __restrict__ partial, unsigned long long* __restrict__ work,
    const double* __restrict__ ut, int64_t ldu, double* __restrict__ atom_part,
    const int32_t* __restrict__ uperm, const int32_t* __restrict__ uptr,
    const int64_t* __restrict__ n_live, int ugroup = 0, int64_t slab0 = 0, int acc_first = -1) {
    // whole workgroups past the real slots leave at once (workgroup-uniform, before any barrier)
    if (n_live && (int64_t)blockIdx.x * blockDim.x >= *n_live) return;
    __shared__ double tab[256];
    __shared__ double af[kAtomF ? 4 : 1][kAtomF ? kAtomChunk : 1][3];
    // Each lane's Ah (6) and centre (3), read again at every new aux centre: held in LDS (one
    // slot per lane, structure of arrays) rather than in registers across the loop.
    __shared__ double geo[9][256];
    for (int i = threadIdx.x; i < 256; i += blockDim.x) tab[i] = exp2_frac_lead(i);
    const int64_t a = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    const bool live = a < (n_live ? *n_live : n);      // n_live: a device count of real slots
    const double* r = rec + kRec * (live ? a : 0);
    const double I1 = r[0], I2 = r[1], I3 = r[2];
#pragma unroll
    for (int c = 0; c < 6; ++c) geo[c][threadIdx.x] = r[3 + c];
    geo[6][threadIdx.x] = live ? r[9] : kFarAway;
    geo[7][threadIdx.x] = live ? r[10] : kFarAway;
    geo[8][threadIdx.x] = live ? r[11] : kFarAway;
    __syncthreads();
    double jt = 0, T1 = 0, T2 = 0, T3 = 0;
    double Vc[3] = {0, 0, 0}, Va[3] = {0, 0, 0}, Vb[3] = {0, 0, 0};
    double Sa[6] = {0, 0, 0, 0, 0, 0}, Sb[6] = {0, 0, 0, 0, 0, 0};
    double C0 = 0, C1 = 0, C2 = 0;
    double d[3] = {0, 0, 0}, q0 = 0, q1 = 0, X0 = 0, rr = 0;
    double ad[3] = {0, 0, 0}, a2d[3] = {0, 0, 0};      // Ah d, Ah^2 d (kAtomF)
    const double cq2 = kAtomF && live ? 2.0 * r[13] * r[14] : 0.0;
    int64_t ut0 = 0;                     // kLaneU: the lane's cotangent rows [ut0, ut0 + utn)
    int utn = 0;
    double uscale = 1.0;                 // kLaneU with ugroup: the group's entry count
    if constexpr (kLaneU) {
        // a dead group (weight 0: coefficient 0) reads no cotangent row: its row may never have
        // been written
        if (live && r[12] != 0.0) {
            const int32_t g = uperm[a];
            if (ugroup) {
                ut0 = g;
                utn = 1;
                uscale = (double)(uptr[g + 1] - uptr[g]);
            } else {
                ut0 = uptr[g];
                utn = uptr[g + 1] - uptr[g];
            }
        }
    }
    const int64_t slab = slab0 + blockIdx.y;       // aux slab of this workgroup
    int64_t chunk0 = slab * per_slab;
    double F = 0, dP0 = 0, dP1 = 0, dP2 = 0, gs1 = 0, gs2 = 0, gs3 = 0;      // node sums
    auto flush = [&]() {
        if constexpr (kFold) {           // the node sums span the centre's records, u folded in
            jt += (q0 == q0) ? F : q0;   // a NaN centre propagates
            T3 += __builtin_fma(q0, -gs1, dP0);
            T2 += dP1;
            T1 += __builtin_fma(q1, -gs2, dP2);
            C0 = -gs1; C1 = -gs2; C2 = -gs3;
            F = 0; dP0 = 0; dP1 = 0; dP2 = 0; gs1 = 0; gs2 = 0; gs3 = 0;
        }
        const double e1x = C1 * d[0], e1y = C1 * d[1], e1z = C1 * d[2];
        const double e2x = C2 * d[0], e2y = C2 * d[1], e2z = C2 * d[2];
        Vc[0] = __builtin_fma(C0, d[0], Vc[0]);
        Vc[1] = __builtin_fma(C0, d[1], Vc[1]);
        Vc[2] = __builtin_fma(C0, d[2], Vc[2]);
        Va[0] += e1x; Va[1] += e1y; Va[2] += e1z;
        Vb[0] += e2x; Vb[1] += e2y; Vb[2] += e2z;
        Sa[0] = __builtin_fma(e1x, d[0], Sa[0]);
        Sa[1] = __builtin_fma(e1y, d[1], Sa[1]);
        Sa[2] = __builtin_fma(e1z, d[2], Sa[2]);
        Sa[3] = __builtin_fma(e1x, d[1], Sa[3]);
        Sa[4] = __builtin_fma(e1x, d[2], Sa[4]);
        Sa[5] = __builtin_fma(e1y, d[2], Sa[5]);
        Sb[0] = __builtin_fma(e2x, d[0], Sb[0]);
        Sb[1] = __builtin_fma(e2y, d[1], Sb[1]);
        Sb[2] = __builtin_fma(e2z, d[2], Sb[2]);
        Sb[3] = __builtin_fma(e2x, d[1], Sb[3]);
        Sb[4] = __builtin_fma(e2x, d[2], Sb[4]);
        Sb[5] = __builtin_fma(e2y, d[2], Sb[5]);
        C0 = 0; C1 = 0; C2 = 0;
    };
    const int64_t p0 = slab * per_slab;
    const int64_t p1 = min(N, p0 + per_slab);
    uint32_t nodes = 0;
    // kLaneU: the lane's summed cotangents of the next kUb records, fetched kUb records at a time
    // (16-byte loads, half a cache line per row, when the rows and the slab start are 16-byte
    // aligned) and shifted down one record per step; each sum adds the rows in order, as one
    // record at a time would. kUb = 4 (a quarter line per refill) was 2.5% slower; 16 (a whole
    // line) cost a wave per SIMD and was 8% slower.
    constexpr int kUb = 8;
    double ub[kUb];
#pragma unroll
    for (int j = 0; j < kUb; ++j) ub[j] = 0.0;
    const bool uvec = kLaneU && (ldu % 2 == 0) && (p0 % 2 == 0) &&
                      (reinterpret_cast<uintptr_t>(ut) % 16 == 0);
    // Each record's centre, u, new-centre flag and node-0 constants are read one record ahead
    // (the first record's here), so their scalar loads overlap a node loop instead of stalling the
    // record's start.
    double c_x = 0, c_y = 0, c_z = 0, c_u = 0, c_s = 0, c_wh = 0, c_s2 = 0, c_is = 0;
    uint64_t c_new = 1;                                  // the flag's bits, tested when used
    if (p0 < p1) {
        const double* __restrict__ xf = aux + kAuxRec * p0;
        c_x = xf[0]; c_y = xf[1]; c_z = xf[2]; c_u = xf[3];
        c_s = xf[rec_s(0)]; c_wh = xf[rec_wh(0)]; c_s2 = xf[rec_s2(0)]; c_is = xf[rec_is(0)];
    }
    for (int64_t p = p0; p < p1; ++p) {
        const double* __restrict__ x = aux + kAuxRec * p;
        const double Rx = c_x, Ry = c_y, Rz = c_z;
        double u = c_u;
        double n_s = c_s, n_wh = c_wh, n_s2 = c_s2, n_is = c_is;
        const bool fresh = c_new != 0;
        if (p + 1 < p1) {                                // wave-uniform
            const double* __restrict__ xn = x + kAuxRec;
            c_x = xn[0]; c_y = xn[1]; c_z = xn[2]; c_u = xn[3];
            c_s = xn[rec_s(0)]; c_wh = xn[rec_wh(0)]; c_s2 = xn[rec_s2(0)]; c_is = xn[rec_is(0)];
            c_new = __builtin_bit_cast(uint64_t, xn[5]);
        }
        if constexpr (kLaneU) {
            if (((p - p0) % kUb) == 0) {                 // wave-uniform
#pragma unroll
                for (int j = 0; j < kUb; ++j) ub[j] = 0.0;
                if (uvec && p + kUb <= p1) {
                    for (int e = 0; e < utn; ++e) {
                        const double2* row = reinterpret_cast<const double2*>(
                            ut + (ut0 + e) * ldu + p);
#pragma unroll
                        for (int j = 0; j < kUb / 2; ++j) {
                            const double2 v = row[j];
                            ub[2 * j] += v.x;
                            ub[2 * j + 1] += v.y;
                        }
                    }
                } else {
                    for (int e = 0; e < utn; ++e) {
                        const double* row = ut + (ut0 + e) * ldu;
#pragma unroll
                        for (int j = 0; j < kUb; ++j)
                            if (p + j < p1) ub[j] += row[p + j];
                    }
                }
            }
            u *= ub[0] * uscale;
#pragma unroll
            for (int j = 0; j + 1 < kUb; ++j) ub[j] = ub[j + 1];
        }
        if (fresh) {                                     // wave-uniform
            flush();
            const int l = threadIdx.x;
            const double xx = geo[0][l], yy = geo[1][l], zz = geo[2][l], xy = geo[3][l],
                         xz = geo[4][l], yz = geo[5][l];
            d[0] = Rx - geo[6][l]; d[1] = Ry - geo[7][l]; d[2] = Rz - geo[8][l];
            const double ax = __builtin_fma(xx, d[0], __builtin_fma(xy, d[1], xz * d[2]));
            const double ay = __builtin_fma(xy, d[0], __builtin_fma(yy, d[1], yz * d[2]));
            const double az = __builtin_fma(xz, d[0], __builtin_fma(yz, d[1], zz * d[2]));
            q0 = __builtin_fma(d[0], d[0], __builtin_fma(d[1], d[1], d[2] * d[2]));
            q1 = __builtin_fma(d[0], ax, __builtin_fma(d[1], ay, d[2] * az));
            const double q2 = __builtin_fma(ax, ax, __builtin_fma(ay, ay, az * az));
            X0 = I3 * q0;
            rr = __builtin_fma(I1, q1, -q2);
            if constexpr (kAtomF) {
                ad[0] = ax; ad[1] = ay; ad[2] = az;
                a2d[0] = __builtin_fma(xx, ax, __builtin_fma(xy, ay, xz * az));
                a2d[1] = __builtin_fma(xy, ax, __builtin_fma(yy, ay, yz * az));
                a2d[2] = __builtin_fma(xz, ax, __builtin_fma(yz, ay, zz * az));
            }
        }
        if constexpr (!kFold) {
            F = 0; dP0 = 0; dP1 = 0; dP2 = 0; gs1 = 0; gs2 = 0; gs3 = 0;
        }
        // each node's constants are read one node ahead, so their scalar load overlaps the
        // previous node's arithmetic
        auto node = [&](auto tc) {
            constexpr int t = decltype(tc)::value;
            const double st = n_s, wh = n_wh, s2 = n_s2, is = n_is;
            if constexpr (t + 1 < kN) {
                n_s = x[rec_s(t + 1)];
                n_wh = x[rec_wh(t + 1)];
                n_s2 = x[rec_s2(t + 1)];
                n_is = x[rec_is(t + 1)];
            }
            const double Pr = __builtin_fma(is, I3, __builtin_fma(st, I1 + st, I2));
            const double Qn = __builtin_fma(st, __builtin_fma(st, q1, rr), X0);
            const NodeValH v = node_val_h(Pr, Qn);
            const double f = (wh * v.y0) * exp_neg_tab_k(v.arg, tab);
            F += f;
            const double G = f * v.ip;                  // g s
            const double Gh = G * v.zh;                 // s df/dPn
            dP0 = __builtin_fma(Gh, is, dP0);
            dP1 += Gh;
            dP2 = __builtin_fma(Gh, st, dP2);
            gs1 += G;
            gs2 = __builtin_fma(G, st, gs2);
            gs3 = __builtin_fma(G, s2, gs3);
            // keep the next node's loads ahead of the early exit (not sunk past it)
            if constexpr (t + 1 < kN)
                asm volatile("" ::"s"(n_s), "s"(n_wh), "s"(n_s2), "s"(n_is));
            return screen_after<kN>(t) && wave_all_beyond_h(v.zh);
        };
        nodes += node_loop<0, kN>(node);
        if constexpr (kFold) continue;
        F = (q0 == q0) ? F : q0;                 // a NaN centre propagates
        jt = __builtin_fma(u, F, jt);
        T3 = __builtin_fma(u, __builtin_fma(q0, -gs1, dP0), T3);
        T2 = __builtin_fma(u, dP1, T2);
        T1 = __builtin_fma(u, __builtin_fma(q1, -gs2, dP2), T1);
        C0 = __builtin_fma(u, -gs1, C0);
        C1 = __builtin_fma(u, -gs2, C1);
        C2 = __builtin_fma(u, -gs3, C2);
        if constexpr (kAtomF) {
            const double f0 = -I3 * gs1, f1 = -__builtin_fma(I1, gs2, gs3), f2 = gs2;
            double fv[3];
#pragma unroll
            for (int c = 0; c < 3; ++c)
                fv[c] = cq2 * __builtin_fma(f0, d[c], __builtin_fma(f1, ad[c], f2 * a2d[c]));
            int comp;
            const double tot = wave_sum3(fv, &comp);
            if (comp >= 0) af[threadIdx.x >> 6][p - chunk0][comp] = tot;
            if (p - chunk0 == kAtomChunk - 1 || p == p1 - 1) {     // workgroup-uniform
                __syncthreads();
                const int i = threadIdx.x / 3, c = threadIdx.x % 3;
                if (threadIdx.x < 3 * kAtomChunk && chunk0 + i <= p)
                    atom_part[((int64_t)blockIdx.x * N + chunk0 + i) * 3 + c] =
                        ((af[0][i][c] + af[1][i][c]) + af[2][i][c]) + af[3][i][c];
                __syncthreads();
                chunk0 = p + 1;
            }
        }
    }
    flush();
    count_work(work, live, nodes);
    if (!live) return;
    double* o = partial + (int64_t)blockIdx.y * kAcc * n + a;
    const double v[kAcc] = {jt, T1, T2, T3, Vc[0], Vc[1], Vc[2], Va[0], Va[1], Va[2],
                            Vb[0], Vb[1], Vb[2], Sa[0], Sa[1], Sa[2], Sa[3], Sa[4], Sa[5],
                            Sb[0], Sb[1], Sb[2], Sb[3], Sb[4], Sb[5]};
    if (acc_first >= 0 && blockIdx.y == 0) {
        // the launch's first slab adds its moments to the running sums of the slabs before it
        // (acc_first: none yet, start from 0), in slab order like a sum over every slab
#pragma unroll
        for (int c = 0; c < kAcc; ++c)
            o[(int64_t)c * n] = (acc_first ? 0.0 : o[(int64_t)c * n]) + v[c];
        return;
    }
#pragma unroll
    for (int c = 0; c < kAcc; ++c) o[(int64_t)c * n] = v[c];
}

// rec_sorted[slot] = rec[perm[slot]].
__global__ void k_rec_gather(int64_t n, const int32_t* __restrict__ perm,
                             const double* __restrict__ rec, double* __restrict__ out) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t >= n * kRec) return;
    const int64_t slot = t / kRec, c = t % kRec;
    out[t] = rec[(int64_t)perm[slot] * kRec + c];
}

__device__ __forceinline__ void sym_mul(const double A[6], const double B[6], double M[9]) {
    // full product of two symmetric matrices in slot form
    const double a[9] = {A[0], A[3], A[4], A[3], A[1], A[5], A[4], A[5], A[2]};
    const double b[9] = {B[0], B[3], B[4], B[3], B[1], B[5], B[4], B[5], B[2]};
    for (int r = 0; r < 3; ++r)
        for (int c = 0; c < 3; ++c)
            M[3 * r + c] = a[3 * r] * b[c] + a[3 * r + 1] * b[3 + c] + a[3 * r + 2] * b[6 + c];
}

__device__ __forceinline__ void sym_vec(const double A[6], const double x[3], double y[3]) {
    y[0] = A[0] * x[0] + A[3] * x[1] + A[4] * x[2];
    y[1] = A[3] * x[0] + A[1] * x[1] + A[5] * x[2];
    y[2] = A[4] * x[0] + A[5] * x[1] + A[2] * x[2];
}

// Reverse of gs_dft/coulomb/stream.py:203-215 for pair a = (i, j): from dE/dAh (Gh, six slots,
// updated in place), dE/dPa (gP) and dE/dKN_a (gKN) to the 20 per-pair splat contributions (SoA):
//   [0..5] G_i  [6..8] g_mu_i  [9] g_N_i  [10..15] G_j  [16..18] g_mu_j  [19] g_N_j.
__device__ void pair_reverse(int64_t n, int64_t a, int64_t i, int64_t j,
                             const double* __restrict__ A6, const double* __restrict__ mu,
                             const double* __restrict__ Nrm, double Gh[6], const double gP[3],
                             double gKN, double* __restrict__ contrib) {
    const Sym3 Ai = load_sym(A6 + 6 * i), Aj = load_sym(A6 + 6 * j);
    const double mui[3] = {mu[3 * i], mu[3 * i + 1], mu[3 * i + 2]};
    const double muj[3] = {mu[3 * j], mu[3 * j + 1], mu[3 * j + 2]};
    const double Ni = Nrm[i], Nj = Nrm[j];
    Sym3 Ahp;
    double Pc[3], KNp;
    pair_quantities(Ai, Aj, mui, muj, Ni, Nj, &Ahp, Pc, &KNp);
    double Gi[6] = {0, 0, 0, 0, 0, 0}, Gj[6] = {0, 0, 0, 0, 0, 0};
    double gmi[3] = {0, 0, 0}, gmj[3] = {0, 0, 0};
    // KN = N_i N_j K, K = exp(-e), e = d . Ai Ah^-1 Aj d
    const double d[3] = {mui[0] - muj[0], mui[1] - muj[1], mui[2] - muj[2]};
    double Ajd[3], Aid[3], u[3], v[3], Aiu[3], Ajv[3];
    matvec(Aj, d, Ajd);
    matvec(Ai, d, Aid);
    solve3(Ahp, Ajd, u);
    solve3(Ahp, Aid, v);
    matvec(Ai, u, Aiu);
    matvec(Aj, v, Ajv);
    const double e = d[0] * Aiu[0] + d[1] * Aiu[1] + d[2] * Aiu[2];
    const double K = exp(-e);
    const double gNi = gKN * Nj * K, gNj = gKN * Ni * K;
    const double ge = -gKN * KNp;
    for (int k = 0; k < 3; ++k) {
        const double gd = ge * (Aiu[k] + Ajv[k]);
        gmi[k] += gd;
        gmj[k] -= gd;
    }
    add_sym_outer(Gi, ge, d, u);
    add_sym_outer(Gj, ge, v, d);
    add_sym_outer(Gh, -ge, v, u);
    // P = Ah^-1 (Ai mu_i + Aj mu_j)
    double y[3];
    solve3(Ahp, gP, y);
    add_sym_outer(Gh, -1.0, y, Pc);
    add_sym_outer(Gi, 1.0, y, mui);
    add_sym_outer(Gj, 1.0, y, muj);
    double Aiy[3], Ajy[3];
    matvec(Ai, y, Aiy);
    matvec(Aj, y, Ajy);
    for (int k = 0; k < 3; ++k) { gmi[k] += Aiy[k]; gmj[k] += Ajy[k]; }
    // Ah = Ai + Aj
    for (int k = 0; k < 6; ++k) { Gi[k] += Gh[k]; Gj[k] += Gh[k]; }
    double out[20];
    for (int k = 0; k < 6; ++k) { out[k] = Gi[k]; out[10 + k] = Gj[k]; }
    for (int k = 0; k < 3; ++k) { out[6 + k] = gmi[k]; out[16 + k] = gmj[k]; }
    out[9] = gNi;
    out[19] = gNj;
    for (int c = 0; c < 20; ++c) contrib[(int64_t)c * n + a] = out[c];
}

// Per pair: sum the slab moments, map them to dE/dAh, dE/dPa, dE/dKN_a, then through
// gs_dft/coulomb/stream.py:203-215 to the two splats. Writes J and 20 contributions (SoA):
//   [0..5] G_i  [6..8] g_mu_i  [9] g_N_i  [10..15] G_j  [16..18] g_mu_j  [19] g_N_j.
// Slot `slot` (of n) holds pair a = perm[slot] (its record and slab moments are stored by slot,
// stride n); J and contrib are indexed by pair, stride nc. pref is the integral's prefactor
// (2 pi^3/sqrt(pi) for (P|a), 2 pi for the nuclear attraction); a null weight treats every entry
// as live.
__global__ void k_pair_finalize(int64_t n, int64_t nc, int64_t slabs, double pref,
                                const int32_t* __restrict__ perm,
                                const int32_t* __restrict__ pi,
                                const int32_t* __restrict__ pj,
                                const double* __restrict__ weight,
                                const double* __restrict__ A6, const double* __restrict__ mu,
                                const double* __restrict__ Nrm, const double* __restrict__ rec,
                                const double* __restrict__ partial, double* __restrict__ J,
                                double* __restrict__ contrib,
                                const int64_t* __restrict__ n_live = nullptr) {
    const int64_t slot = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (slot >= (n_live ? *n_live : n)) return;       // n_live: a device count of real slots
    const int64_t a = perm[slot];
    if (weight && weight[a] == 0.0) {
        J[a] = 0.0;
        for (int c = 0; c < 20; ++c) contrib[(int64_t)c * nc + a] = 0.0;
        return;
    }
    double m[kAcc];
    for (int c = 0; c < kAcc; ++c) {
        double s = 0.0;
        for (int64_t k = 0; k < slabs; ++k) s += partial[(k * kAcc + c) * n + slot];
        m[c] = s;
    }
    const double* r = rec + kRec * slot;
    const double I1 = r[0], I3 = r[2];
    const double Ah[6] = {r[3], r[4], r[5], r[6], r[7], r[8]};
    const double KN = r[13], q = r[14];
    const double jt = m[0], T1 = m[1], T2 = m[2], T3 = m[3];
    const double* Vc = m + 4;
    const double* Va = m + 7;
    const double* Vb = m + 10;
    const double* Sa = m + 13;
    const double* Sb = m + 19;
    const double scale = q * KN * pref;
    J[a] = KN * pref * jt;
    const double gKN = q * pref * jt;
    // dE/dPa = -2 scale (I3 Vc + Ah (I1 Va + Vb) - Ah (Ah Va))
    double w1[3] = {I1 * Va[0] + Vb[0], I1 * Va[1] + Vb[1], I1 * Va[2] + Vb[2]};
    double t1[3], t2[3], t3[3];
    sym_vec(Ah, w1, t1);
    sym_vec(Ah, Va, t2);
    sym_vec(Ah, t2, t3);
    double gP[3];
    for (int k = 0; k < 3; ++k) gP[k] = -2.0 * scale * (I3 * Vc[k] + t1[k] - t3[k]);
    // dE/dAh = scale ((I1 Sa + Sb) - (Ah Sa + Sa Ah) + T1 I + T2 (I1 I - Ah) + T3 adj(Ah))
    double AS[9];
    sym_mul(Ah, Sa, AS);
    const Sym3 AhS{Ah[0], Ah[1], Ah[2], Ah[3], Ah[4], Ah[5]};
    double adj[9];
    adj3(AhS, adj);
    const int rr_[6] = {0, 1, 2, 0, 0, 1}, cc_[6] = {0, 1, 2, 1, 2, 2};
    double Gh[6];
    for (int k = 0; k < 6; ++k) {
        const int rw = rr_[k], cl = cc_[k];
        const double eye = (rw == cl) ? 1.0 : 0.0;
        Gh[k] = scale * ((I1 * Sa[k] + Sb[k]) - (AS[3 * rw + cl] + AS[3 * cl + rw]) + T1 * eye
                         + T2 * (I1 * eye - Ah[k]) + T3 * adj[3 * rw + cl]);
    }
    pair_reverse(nc, a, pi[a], pj[a], A6, mu, Nrm, Gh, gP, gKN, contrib);
}

// One wave per splat: deterministic segmented sums of the i-side and j-side contributions, then
// the chart reverse (gs_dft/basis/spectral.py:33-40,72-82).
__global__ __launch_bounds__(256) void k_splat_grad(
    int64_t M, int64_t n, const int32_t* __restrict__ row_ptr, const int32_t* __restrict__ row_perm,
    const int32_t* __restrict__ col_ptr, const int32_t* __restrict__ col_perm,
    const double* __restrict__ contrib, const double* __restrict__ quat,
    const double* __restrict__ log_scale, double* __restrict__ dquat,
    double* __restrict__ dlog_scale, double* __restrict__ dcenters) {
    const int64_t m = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (m >= M) return;
    double acc[10];
    for (int c = 0; c < 10; ++c) acc[c] = 0.0;
    for (int64_t p = row_ptr[m] + lane; p < row_ptr[m + 1]; p += 64) {
        const int64_t a = row_perm[p];
        for (int c = 0; c < 10; ++c) acc[c] += contrib[(int64_t)c * n + a];
    }
    for (int64_t p = col_ptr[m] + lane; p < col_ptr[m + 1]; p += 64) {
        const int64_t a = col_perm[p];
        for (int c = 0; c < 10; ++c) acc[c] += contrib[(int64_t)(10 + c) * n + a];
    }
    for (int c = 0; c < 10; ++c) acc[c] = wave_sum(acc[c]);
    if (lane != 0) return;
    chart_reverse(m, acc, quat, log_scale, dquat, dlog_scale, dcenters);
}

// dE/dC_mo = occ_o [sum_{a: i_a=m} J_a w_a C_{j_a o} + sum_{a: j_a=m} J_a w_a C_{i_a o}]
// (gs_dft/coulomb/ri.py:456 reverse). The orbitals are cut into chunks of 256 CH, one workgroup
// per (chunk, splat), thread t owning orbitals o = base + t + 256 c (c < CH) and streaming the
// partners' chunk rows coalesced. The splat's pairs (its CSR row, then its column) are taken 256
// at a time: each thread resolves one pair's partner and scale J_a w_a into LDS, so the streaming
// loop carries no dependent index loads. The logical blocks run chunk-major and XCD-contiguously,
// so the workgroups of one XCD walk consecutive splats (the splats of one atom, which share most
// of their partners) for one chunk and find part of those rows in that XCD's L2: 32.0 ms at the
// 700-atom globule against 36.0 ms with whole rows per workgroup (512-orbital chunks: 32.9 ms).
// Each output element is summed by one thread over the pairs in CSR order.
template <int CH>
__global__ __launch_bounds__(256) void k_dC(int64_t M, int64_t k, int64_t nchunks,
                                            const int32_t* __restrict__ row_ptr,
                                            const int32_t* __restrict__ row_perm,
                                            const int32_t* __restrict__ col_ptr,
                                            const int32_t* __restrict__ col_perm,
                                            const int32_t* __restrict__ pi,
                                            const int32_t* __restrict__ pj,
                                            const double* __restrict__ J,
                                            const double* __restrict__ weight,
                                            const double* __restrict__ C,
                                            const double* __restrict__ occ,
                                            double* __restrict__ dC) {
    __shared__ int32_t partner[256];
    __shared__ double scale[256];
    const int64_t lb = xcd_block(M * nchunks);
    if (lb < 0) return;                          // workgroup-uniform
    const int64_t m = lb % M, base = (lb / M) * (256 * CH);
    const int64_t r0 = row_ptr[m], r1 = row_ptr[m + 1], c0 = col_ptr[m], c1 = col_ptr[m + 1];
    const int64_t nr = r1 - r0, total = nr + (c1 - c0);
    double acc[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) acc[c] = 0.0;
    for (int64_t b0 = 0; b0 < total; b0 += 256) {
        const int64_t e = b0 + threadIdx.x;
        if (e < total) {
            const int64_t a = e < nr ? row_perm[r0 + e] : col_perm[c0 + e - nr];
            partner[threadIdx.x] = e < nr ? pj[a] : pi[a];
            scale[threadIdx.x] = J[a] * weight[a];
        }
        __syncthreads();
        const int cnt = (int)min((int64_t)256, total - b0);
        for (int q = 0; q < cnt; ++q) {
            const double sc = scale[q];
            const double* __restrict__ row = C + (int64_t)partner[q] * k;
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const int64_t o = base + threadIdx.x + 256 * c;
                if (o < k) acc[c] = __builtin_fma(sc, row[o], acc[c]);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int64_t o = base + threadIdx.x + 256 * c;
        if (o < k) dC[m * k + o] = occ[o] * acc[c];
    }
}

// ------------------------------------------------------------------ nuclear attraction
// gs_dft/screening/pairs.py:348-370: V_a = -N_i N_j K sum_A Z_A (2/sqrt(pi)) sum_t w_t pi^1.5
// det(B_t)^(-1/2) exp(-(t^2 |d|^2 - t^4 d.adj(B_t) d / det B_t)), B_t = Ah + t^2 I, d = Pa - R_A.
// With s = t^2: det B_t = Pn(s) and the exponent is s d.Ah (Ah + s I)^-1 d = s Qn(s)/Pn(s), the
// three-centre node of an aux function whose exponent b grows without bound (s_t = t^2 b/(b + t^2)
// -> t^2, w_t (b + t^2)^(-3/2) -> w_t once the aux norm is divided out). So the nuclei enter the
// reverse kernel as aux records with s_t = t^2, wp_t = w_t and u = -Z_A, and the prefactor is
// (2/sqrt(pi)) pi^1.5 = 2 pi.
constexpr double kPrefNuc = 2.0 * kPi;

__global__ void k_atom_rec(int64_t n_atoms, const double* __restrict__ coords,
                           const double* __restrict__ charges, double* __restrict__ out) {
    const int64_t A = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (A >= n_atoms) return;
    double* o = out + kAuxRec * A;
    o[0] = coords[3 * A]; o[1] = coords[3 * A + 1]; o[2] = coords[3 * A + 2];
    o[3] = -charges[A];
    bool first = true;
    if (A > 0)
        first = !(__builtin_bit_cast(uint64_t, coords[3 * A - 3]) ==
                      __builtin_bit_cast(uint64_t, coords[3 * A]) &&
                  __builtin_bit_cast(uint64_t, coords[3 * A - 2]) ==
                      __builtin_bit_cast(uint64_t, coords[3 * A + 1]) &&
                  __builtin_bit_cast(uint64_t, coords[3 * A - 1]) ==
                      __builtin_bit_cast(uint64_t, coords[3 * A + 2]));
    o[4] = 0.0; o[5] = first ? 1.0 : 0.0; o[6] = 0.0; o[7] = 0.0;
    for (int t = 0; t < kNodes; ++t) put_node_consts(o, t, quad_t(t) * quad_t(t), quad_w(t));
}

// ------------------------------------------------------------------ exact pair-pair Coulomb
// gs_dft/coulomb/stream.py:249-281,296-320: (a|b) = KN_a KN_b (2/sqrt(pi)) sum_t w_t pi^3
// det(G_t)^(-1/2) exp(-quad_t), G_t the 6x6 block precision [[A_a + sI, -sI], [-sI, A_b + sI]]
// at s = t^2 (the reference reduces it by a Schur complement). With T = A_a^-1 + A_b^-1 and
// d = P_a - P_b, det G_t = det A_a det A_b det(I + sT) and quad_t = s d.(I + sT)^-1 d, and
// Cayley-Hamilton gives, division-free,
//   E(s) = det(I + sT) = 1 + s (J1 + s (J2 + s J3)),  J1 = tr T, J2 = tr adj T, J3 = det T,
//   s d.adj(I + sT).d = s (p0 + s (p1 + s p2)),     p0 = |d|^2, p1 = J1 p0 - d.T d, p2 = d.adj T.d,
// so (a|b) = h_a h_b 2 pi^2.5 sum_t w_t E^(-1/2) e^(-z), z = s (p0 + s p1 + s^2 p2) / E, with
// h = KN det(A)^(-1/2) per pair -- the node of the three-centre kernels with s_t = t^2.
// Pair record (slot order): A^-1 (6) | P (3) | h | Pw (= w sum_o occ_o C_io C_jo, or w P_ij) | w.
constexpr int kEriRec = 12;
constexpr double kPrefEri = kTwoPi25;                 // (2/sqrt(pi)) pi^3 = 2 pi^2.5

__global__ void k_eri_rec(int64_t n, const int32_t* __restrict__ perm,
                          const int32_t* __restrict__ pi, const int32_t* __restrict__ pj,
                          const double* __restrict__ A6, const double* __restrict__ mu,
                          const double* __restrict__ Nrm, const double* __restrict__ q,
                          const double* __restrict__ weight, double* __restrict__ rec) {
    const int64_t slot = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (slot >= n) return;
    const int64_t a = perm[slot];
    const int64_t i = pi[a], j = pj[a];
    const Sym3 Ai = load_sym(A6 + 6 * i), Aj = load_sym(A6 + 6 * j);
    const double mui[3] = {mu[3 * i], mu[3 * i + 1], mu[3 * i + 2]};
    const double muj[3] = {mu[3 * j], mu[3 * j + 1], mu[3 * j + 2]};
    Sym3 Ah;
    double P[3], KN;
    pair_quantities(Ai, Aj, mui, muj, Nrm[i], Nrm[j], &Ah, P, &KN);
    double c[9];
    adj3(Ah, c);
    const double det = det3(Ah);
    double* r = rec + kEriRec * slot;
    r[0] = c[0] / det; r[1] = c[4] / det; r[2] = c[8] / det;
    r[3] = c[1] / det; r[4] = c[2] / det; r[5] = c[5] / det;
    r[6] = P[0]; r[7] = P[1]; r[8] = P[2];
    r[9] = KN / sqrt(det);
    r[10] = q[a];
    r[11] = weight ? weight[a] : 1.0;
}

// The centre-dependent scalars of one pair-pair from T (six slots) and d.
struct EriGeom {
    double J1, J2, J3, p0, p1, p2;
};

__device__ __forceinline__ EriGeom eri_geom(const double T[6], const double d[3], double adjT[6],
                                           double Td[3]) {
    const double xx = T[0], yy = T[1], zz = T[2], xy = T[3], xz = T[4], yz = T[5];
    adjT[0] = __builtin_fma(yy, zz, -yz * yz);
    adjT[1] = __builtin_fma(xx, zz, -xz * xz);
    adjT[2] = __builtin_fma(xx, yy, -xy * xy);
    adjT[3] = __builtin_fma(xz, yz, -xy * zz);
    adjT[4] = __builtin_fma(xy, yz, -xz * yy);
    adjT[5] = __builtin_fma(xy, xz, -xx * yz);
    EriGeom g;
    g.J1 = xx + yy + zz;
    g.J2 = adjT[0] + adjT[1] + adjT[2];
    g.J3 = __builtin_fma(xx, adjT[0], __builtin_fma(xy, adjT[3], xz * adjT[4]));
    Td[0] = __builtin_fma(xx, d[0], __builtin_fma(xy, d[1], xz * d[2]));
    Td[1] = __builtin_fma(xy, d[0], __builtin_fma(yy, d[1], yz * d[2]));
    Td[2] = __builtin_fma(xz, d[0], __builtin_fma(yz, d[1], zz * d[2]));
    g.p0 = __builtin_fma(d[0], d[0], __builtin_fma(d[1], d[1], d[2] * d[2]));
    const double dTd = __builtin_fma(d[0], Td[0], __builtin_fma(d[1], Td[1], d[2] * Td[2]));
    g.p1 = __builtin_fma(g.J1, g.p0, -dTd);
    const double ax = __builtin_fma(adjT[0], d[0], __builtin_fma(adjT[3], d[1], adjT[4] * d[2]));
    const double ay = __builtin_fma(adjT[3], d[0], __builtin_fma(adjT[1], d[1], adjT[5] * d[2]));
    const double az = __builtin_fma(adjT[4], d[0], __builtin_fma(adjT[5], d[1], adjT[2] * d[2]));
    g.p2 = __builtin_fma(d[0], ax, __builtin_fma(d[1], ay, d[2] * az));
    return g;
}

// Sums of ten values over the 64 lanes of a wave by a transposing butterfly: at the exchanges
// that pair lanes across bit 5 (swap32), bit 4 (swap16), bit 3 (row mirror) and bit 2 (half-row
// mirror) of the lane index each lane keeps half of its partial sums and trades the other half
// (5, 3, 2, 1 values), then two quad permutes finish. The total of value (b5 ? 5 : 0) + slot,
// slot = (b4 ? 3 : 0) + (b3 ? 2 : 0) + b2, ends in the lanes with bits 1, 0 clear; returns it and
// sets *idx to the value's index on the ten such lanes that hold one, -1 elsewhere. The
// summation order is fixed.
__device__ __forceinline__ double wave_sum10(const double v[10], int* idx) {
    const int L = threadIdx.x & 63;
    const bool b4 = L & 16, b3 = L & 8, b2 = L & 4;
    double u[6];
#pragma unroll
    for (int i = 0; i < 5; ++i) {
        double x = v[i], y = v[5 + i];
        swap32(x, y);
        u[i] = x + y;
    }
    u[5] = 0.0;
    double w[4];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        double x = u[j], y = u[3 + j];
        swap16(x, y);
        w[j] = x + y;
    }
    w[3] = 0.0;
    double xk[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const double send = b3 ? w[k] : w[2 + k], keep = b3 ? w[2 + k] : w[k];
        xk[k] = keep + dpp<0x140>(send);
    }
    const double send = b2 ? xk[0] : xk[1], keep = b2 ? xk[1] : xk[0];
    double y = keep + dpp<0x141>(send);
    y += dpp<0x4e>(y);
    y += dpp<0xb1>(y);
    const int bslot = (b3 ? 2 : 0) + (b2 ? 1 : 0);
    const int aslot = (b4 ? 3 : 0) + bslot;
    *idx = ((L & 3) == 0 && bslot <= 2 && aslot <= 4) ? ((L & 32) ? 5 : 0) + aslot : -1;
    return y;
}

// Sum of v over the 64 lanes of a wave, in every lane, by the same exchanges as wave_sum10
// (fixed order).
__device__ __forceinline__ double wave_sum_x(double v) {
    double x = v, y = v;
    swap32(x, y);
    v = x + y;
    x = v; y = v;
    swap16(x, y);
    v = x + y;
    v += dpp<0x140>(v);
    v += dpp<0x141>(v);
    v += dpp<0x4e>(v);
    v += dpp<0xb1>(v);
    return v;
}

// Symmetric forward over one band of bra slots [A0, A0 + H): (a|b) = (b|a), so each unordered
// pair-pair is evaluated once, in the workgroup whose bra lanes hold a and whose ket slab holds
// b >= a (a == b once, as a bra term). The bra lane accumulates c_b F_ab (c = h Pw); the ket
// side c_a F_ab is summed over the wave's lanes (wave_sum_x) for every ket,
// kept per wave in LDS and written per workgroup (the four waves added in order) to
// ket_part[x][b - A0] for the whole slab (zeros where a wave had no ket). Lanes with a > b (only
// near the diagonal) contribute nothing and do not hold the wave in the node loop.
// 768 kets per workgroup: the per-wave ket sums then take 24 KB of LDS, so the kernel runs the
// five waves per SIMD its registers allow (1024 kets, 32 KB: four, 1.9% slower).
constexpr int kEriSymSlab = 768;

__global__ __launch_bounds__(256) void k_eri_fwd_sym(int64_t n, const double* __restrict__ rec,
                                                     int64_t A0, int64_t H,
                                                     double* __restrict__ bra_part,
                                                     double* __restrict__ ket_part,
                                                     unsigned long long* __restrict__ work) {
    __shared__ double tab[256];
    __shared__ double kw[4][kEriSymSlab];
    for (int i = threadIdx.x; i < 256; i += blockDim.x) tab[i] = exp2_frac_lead(i);
    for (int i = threadIdx.x; i < 4 * kEriSymSlab; i += blockDim.x) (&kw[0][0])[i] = 0.0;
    __syncthreads();
    const int wv = threadIdx.x >> 6;
    const int64_t a = A0 + (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t band_end = min(n, A0 + H);
    const bool live = a < band_end;
    const double* __restrict__ ra = rec + kEriRec * (live ? a : 0);
    const double Ta[6] = {ra[0], ra[1], ra[2], ra[3], ra[4], ra[5]};
    const double Px = live ? ra[6] : kFarAway, Py = live ? ra[7] : kFarAway,
                 Pz = live ? ra[8] : kFarAway;
    const double ca = live ? ra[9] * ra[10] : 0.0;
    const int64_t kb0 = A0 + (int64_t)blockIdx.y * kEriSymSlab;
    const int64_t kb1 = min(n, kb0 + kEriSymSlab);
    const int64_t amin = A0 + (int64_t)blockIdx.x * 256 + wv * 64;
    const double c256 = vgpr_const(kNegC256);
    double acc = 0.0;
    uint32_t nodes = 0;
    auto ket = [&](int64_t b, auto maskc) {
        constexpr bool kMask = decltype(maskc)::value;
        const double* __restrict__ rb = rec + kEriRec * b;
        const double cb = rb[9] * rb[10];              // h_b Pw_b, wave-uniform
        if (cb == 0.0) return;                         // padding and zero weights: J_b is not used
        const bool off = kMask && a > b;               // this lane's pair-pair is another's
        const double T[6] = {Ta[0] + rb[0], Ta[1] + rb[1], Ta[2] + rb[2],
                             Ta[3] + rb[3], Ta[4] + rb[4], Ta[5] + rb[5]};
        const double d[3] = {Px - rb[6], Py - rb[7], Pz - rb[8]};
        double adjT[6], Td[3];
        const EriGeom G = eri_geom(T, d, adjT, Td);
        double F = 0.0;
        // the node weight rides in the exponent as in the DF-J forward (exp_neg_tab_k_w); the
        // split of the compile-time weight folds to constants
        auto node = [&](auto tc) {
            constexpr int t = decltype(tc)::value;
            constexpr double st = quad_t(t) * quad_t(t), is = 1.0 / st;
            constexpr double wh = quad_w(t) / quad_t(t) * (kExpMinusHalf / kExpPolyK);
            double S;
            double lw = fold_weight(wh, &S);
            // materialised in scalar registers at each node (not held in vector registers
            // across the ket loop)
            asm volatile("" : "+s"(lw), "+s"(S));
            const double Er = __builtin_fma(st, __builtin_fma(st, G.J3, G.J2), G.J1) + is;
            const double num = __builtin_fma(st, __builtin_fma(st, G.p2, G.p1), G.p0);
            const double y0 = __builtin_amdgcn_rsq(Er);
            const double h = y0 * y0;
            const double e1 = __builtin_fma(-Er, h, 2.0);
            const double za = __builtin_fma(num, h, -0.5);
            F = __builtin_fma(y0, exp_neg_tab_k_w(__builtin_fma(za, e1, lw), S, c256, tab), F);
            if constexpr (kMask)
                return screen_after(t) && wave_all_beyond_h(off ? kFarAway : za);
            else
                return screen_after(t) && wave_all_beyond_h(za);
        };
        nodes += node_loop<0>(node);
        F = (G.p0 == G.p0) ? F : G.p0;                 // a NaN centre propagates
        if (!off) acc = __builtin_fma(F, cb, acc);
        const double ks = wave_sum_x((off || a == b) ? 0.0 : ca * F);
        if ((threadIdx.x & 63) == 0) kw[wv][b - kb0] = ks;
    };
    int64_t b = kb0 > amin ? kb0 : amin;
    for (; b < kb1 && b < amin + 64; ++b) ket(b, std::true_type{});
    for (; b < kb1; ++b) ket(b, std::false_type{});
    count_work(work, live, nodes);
    __syncthreads();
    double* kp = ket_part + (int64_t)blockIdx.x * (n - A0) + (kb0 - A0);
    for (int i = threadIdx.x; i < kb1 - kb0; i += blockDim.x)
        kp[i] = ((kw[0][i] + kw[1][i]) + kw[2][i]) + kw[3][i];
    if (live) bra_part[(int64_t)blockIdx.y * H + (a - A0)] = acc;
}

// Jacc[b] += sum_x ket_part[x][b - A0] (x in order) and, for b in the band, + sum_y
// bra_part[y][b - A0] (y in order): the band's share of sum_b' c_b' F_bb'.
__global__ void k_eri_sym_reduce(int64_t n, int64_t A0, int64_t H, int64_t groups, int64_t slabs,
                                 int64_t acc_stride, const double* __restrict__ bra_part,
                                 const double* __restrict__ ket_part, double* __restrict__ Jacc) {
    const int64_t b = A0 + blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (b >= n) return;
    double s = 0.0;
    for (int64_t x = 0; x < groups; ++x) s += ket_part[x * (n - A0) + (b - A0)];
    if (b < A0 + H)
        for (int64_t y = 0; y < slabs; ++y) s += bra_part[y * acc_stride + (b - A0)];
    Jacc[b] += s;
}

// Reverse moments of a pair a: MJ = sum_b c_b F, MT = sum_b c_b dF/dT (six slots) and
// Md = sum_b c_b dF/dd, c_b = h_b Pw_b.
//   node sums: F, A_k = sum g (z - 1/2) s^k, B_k = sum g s^k (k = 1..3), g = f / E;
//   dF/dJ_k = A_k, dF/dp_k = -B_(k+1); with p1 = J1 p0 - d.T d and p2 = |T d|^2 - J1 d.T d + J2 p0:
//   dF/dT = gJ1 I + gJ2 (J1 I - T) + gJ3 adj T - gp1' d d^T
//           + gp2 ((T d d^T + d d^T T) - (d.T d) I - J1 d d^T + p0 (J1 I - T)),
//   dF/dd = 2 (gp0' d + gp1'' T d + gp2 adj(T) d), primes folding the p1 chain.
constexpr int kEriAcc = 10;

// Symmetric reverse over one band of bra slots [A0, A0 + H), as k_eri_fwd_sym: each unordered
// pair-pair once. Per pair-pair the node sums and the chain above give F, gT = dF/dT (six
// slots) and gd = dF/dd (d = P_a - P_b); the bra lane accumulates c_b (F, gT, gd),
// and the ket's moments c_a (F, gT, -gd) (T is symmetric in a and b, d changes sign) are summed over
// the wave (wave_sum10) and written per wave to ket_part[(4 x + wave) * 10 + c][b - A0] for every
// ket of the workgroup's slab (zeros where the wave had no ket).
// kets per workgroup of the reverse: the forward's, so that both passes sum the bra partials of
// a band over the same slabs and their E_J agree bit for bit
constexpr int kEriSymSlabB = kEriSymSlab;

__global__ __launch_bounds__(256) void k_eri_bwd_sym(int64_t n, const double* __restrict__ rec,
                                                     int64_t A0, int64_t H,
                                                     double* __restrict__ bra_part,
                                                     double* __restrict__ ket_part,
                                                     unsigned long long* __restrict__ work) {
    __shared__ double tab[256];
    for (int i = threadIdx.x; i < 256; i += blockDim.x) tab[i] = exp2_frac_lead(i);
    __syncthreads();
    const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t a = A0 + (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t band_end = min(n, A0 + H);
    const bool live = a < band_end;
    const double* __restrict__ ra = rec + kEriRec * (live ? a : 0);
    const double Ta[6] = {ra[0], ra[1], ra[2], ra[3], ra[4], ra[5]};
    const double Px = live ? ra[6] : kFarAway, Py = live ? ra[7] : kFarAway,
                 Pz = live ? ra[8] : kFarAway;
    const double ca = live ? ra[9] * ra[10] : 0.0;
    const int64_t kb0 = A0 + (int64_t)blockIdx.y * kEriSymSlabB;
    const int64_t kb1 = min(n, kb0 + kEriSymSlabB);
    const int64_t amin = A0 + (int64_t)blockIdx.x * 256 + wv * 64;
    const int64_t nk = n - A0;
    double* __restrict__ kp = ket_part + ((int64_t)blockIdx.x * 4 + wv) * kEriAcc * nk;
    // kets before the wave's first bra: zeros
    for (int64_t b = kb0 + lane; b < kb1 && b < amin; b += 64)
        for (int c = 0; c < kEriAcc; ++c) kp[c * nk + (b - A0)] = 0.0;
    double MJ = 0.0, MT[6] = {0, 0, 0, 0, 0, 0}, Md[3] = {0, 0, 0};
    uint32_t nodes = 0;
    auto ket = [&](int64_t b, auto maskc) {
        constexpr bool kMask = decltype(maskc)::value;
        const double* __restrict__ rb = rec + kEriRec * b;
        const double cb = rb[9] * rb[10];
        if (cb == 0.0) {                               // no moments needed for this ket
            if (lane < kEriAcc) kp[lane * nk + (b - A0)] = 0.0;
            return;
        }
        const bool off = kMask && a > b;
        const double T[6] = {Ta[0] + rb[0], Ta[1] + rb[1], Ta[2] + rb[2],
                             Ta[3] + rb[3], Ta[4] + rb[4], Ta[5] + rb[5]};
        const double d[3] = {Px - rb[6], Py - rb[7], Pz - rb[8]};
        double adjT[6], Td[3];
        const EriGeom G = eri_geom(T, d, adjT, Td);
        double F = 0, A1 = 0, A2 = 0, A3 = 0, B1 = 0, B2 = 0, B3 = 0;
        auto node = [&](auto tc) {
            constexpr int t = decltype(tc)::value;
            constexpr double st = quad_t(t) * quad_t(t), is = 1.0 / st;
            constexpr double wh = quad_w(t) / quad_t(t) * (kExpMinusHalf / kExpPolyK);
            const double Er = __builtin_fma(st, __builtin_fma(st, G.J3, G.J2), G.J1) + is;
            const double num = __builtin_fma(st, __builtin_fma(st, G.p2, G.p1), G.p0);
            const NodeValH v = node_val_h(Er, num);
            const double f = (wh * v.y0) * exp_neg_tab_k(v.arg, tab);
            F += f;
            const double gs = f * v.ip;                 // g s, g = f / Es
            const double ghs = gs * v.zh;               // gh s, gh = g (z - 1/2)
            A1 += ghs;
            A2 = __builtin_fma(ghs, st, A2);
            A3 = __builtin_fma(ghs, st * st, A3);
            B1 += gs;
            B2 = __builtin_fma(gs, st, B2);
            B3 = __builtin_fma(gs, st * st, B3);
            if constexpr (kMask)
                return screen_after(t) && wave_all_beyond_h(off ? kFarAway : v.zh);
            else
                return screen_after(t) && wave_all_beyond_h(v.zh);
        };
        nodes += node_loop<0>(node);
        F = (G.p0 == G.p0) ? F : G.p0;
        const double gp1 = -B2, gp2 = -B3;
        const double gJ1 = __builtin_fma(gp1, G.p0, A1);
        const double gp0 = __builtin_fma(gp1, G.J1, -B1);
        const double gJ2 = A2, gJ3 = A3;
        const double dTd = __builtin_fma(d[0], Td[0], __builtin_fma(d[1], Td[1], d[2] * Td[2]));
        const double diag = gJ1 + G.J1 * __builtin_fma(gp2, G.p0, gJ2) - gp2 * dTd;
        const double cT = -__builtin_fma(gp2, G.p0, gJ2);
        const double cdd = -__builtin_fma(gp2, G.J1, gp1);
        const int rr_[6] = {0, 1, 2, 0, 0, 1}, cc_[6] = {0, 1, 2, 1, 2, 2};
        double gT[6];
#pragma unroll
        for (int k = 0; k < 6; ++k) {
            const int r = rr_[k], c = cc_[k];
            double gt = __builtin_fma(cT, T[k], gJ3 * adjT[k]);
            gt = __builtin_fma(cdd, d[r] * d[c], gt);
            gt = __builtin_fma(gp2, __builtin_fma(Td[r], d[c], d[r] * Td[c]), gt);
            if (r == c) gt += diag;
            gT[k] = gt;
        }
        const double ax = __builtin_fma(adjT[0], d[0], __builtin_fma(adjT[3], d[1], adjT[4] * d[2]));
        const double ay = __builtin_fma(adjT[3], d[0], __builtin_fma(adjT[1], d[1], adjT[5] * d[2]));
        const double az = __builtin_fma(adjT[4], d[0], __builtin_fma(adjT[5], d[1], adjT[2] * d[2]));
        const double gd[3] = {2.0 * __builtin_fma(gp0, d[0], __builtin_fma(-gp1, Td[0], gp2 * ax)),
                              2.0 * __builtin_fma(gp0, d[1], __builtin_fma(-gp1, Td[1], gp2 * ay)),
                              2.0 * __builtin_fma(gp0, d[2], __builtin_fma(-gp1, Td[2], gp2 * az))};
        const double cbra = off ? 0.0 : cb;
        MJ = __builtin_fma(F, cbra, MJ);
#pragma unroll
        for (int k = 0; k < 6; ++k) MT[k] = __builtin_fma(cbra, gT[k], MT[k]);
#pragma unroll
        for (int k = 0; k < 3; ++k) Md[k] = __builtin_fma(cbra, gd[k], Md[k]);
        const double cket = (off || a == b) ? 0.0 : ca;
        const double v[kEriAcc] = {cket * F, cket * gT[0], cket * gT[1], cket * gT[2],
                                   cket * gT[3], cket * gT[4], cket * gT[5],
                                   -cket * gd[0], -cket * gd[1], -cket * gd[2]};
        int idx;
        const double tot = wave_sum10(v, &idx);
        if (idx >= 0) kp[idx * nk + (b - A0)] = tot;
    };
    int64_t b = kb0 > amin ? kb0 : amin;
    for (; b < kb1 && b < amin + 64; ++b) ket(b, std::true_type{});
    for (; b < kb1; ++b) ket(b, std::false_type{});
    count_work(work, live, nodes);
    if (!live) return;
    double* o = bra_part + (int64_t)blockIdx.y * kEriAcc * H + (a - A0);
    const double mv[kEriAcc] = {MJ, MT[0], MT[1], MT[2], MT[3], MT[4], MT[5], Md[0], Md[1], Md[2]};
#pragma unroll
    for (int c = 0; c < kEriAcc; ++c) o[(int64_t)c * H] = mv[c];
}

// The band's share of every pair's ten reverse moments, in a fixed order: first
// macc[c][b] += sum_x ket_part[x * 10 + c][b - A0] (x in order) for every b >= A0 (one thread per b),
// then macc[c][b] += sum_y bra_part[y * 10 + c][b - A0] (y in order) for b in the band (one thread per
// (c, b)).
__global__ void k_eri_sym_reduce10_ket(int64_t n, int64_t A0, int64_t waves,
                                       const double* __restrict__ ket_part,
                                       double* __restrict__ macc) {
    const int64_t b = A0 + blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (b >= n) return;
    const int64_t nk = n - A0;
#pragma unroll
    for (int c = 0; c < kEriAcc; ++c) {
        double s = 0.0;
        for (int64_t x = 0; x < waves; ++x) s += ket_part[(x * kEriAcc + c) * nk + (b - A0)];
        macc[(int64_t)c * n + b] += s;
    }
}

__global__ void k_eri_sym_reduce10_bra(int64_t n, int64_t A0, int64_t H, int64_t slabs,
                                       const double* __restrict__ bra_part,
                                       double* __restrict__ macc) {
    const int64_t hb = min(H, n - A0);
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t >= kEriAcc * hb) return;
    const int64_t c = t / hb, i = t % hb;
    double s = 0.0;
    for (int64_t y = 0; y < slabs; ++y) s += bra_part[(y * kEriAcc + c) * H + i];
    macc[c * n + A0 + i] += s;
}

// J[perm[slot]] = h_a 2 pi^2.5 sum_slabs Jpart (0 on zero-weight entries).
__global__ void k_eri_finish(int64_t n, int64_t slabs, const int32_t* __restrict__ perm,
                             const double* __restrict__ rec, const double* __restrict__ partial,
                             double* __restrict__ J) {
    const int64_t slot = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (slot >= n) return;
    const double* r = rec + kEriRec * slot;
    double acc = 0.0;
    for (int64_t k = 0; k < slabs; ++k) acc += partial[k * n + slot];
    J[perm[slot]] = (r[11] == 0.0) ? 0.0 : r[9] * kPrefEri * acc;     // 0 on dead entries
}

// Per slot: J and the pair's gradient from the reverse moments. E = 1/2 sum_ab Pw_a Pw_b (a|b), so
// dE/dh_a = Pw_a pref MJ, dE/dT_a = Pw_a h_a pref MT (T = A_a^-1 + A_b^-1, so dE/dA_a =
// -A^-1 (dE/dT_a) A^-1), dE/dP_a = Pw_a h_a pref Md; h = KN det(A)^(-1/2) adds
// dE/dKN = gh det(A)^(-1/2) and dE/dA = -gh h A^-1 / 2. Then the pair reverse to the two splats.
__global__ void k_eri_finalize(int64_t n, int64_t slabs, const int32_t* __restrict__ perm,
                               const int32_t* __restrict__ pi, const int32_t* __restrict__ pj,
                               const double* __restrict__ A6, const double* __restrict__ mu,
                               const double* __restrict__ Nrm, const double* __restrict__ rec,
                               const double* __restrict__ partial, double* __restrict__ J,
                               double* __restrict__ contrib) {
    const int64_t slot = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (slot >= n) return;
    const int64_t a = perm[slot];
    const double* r = rec + kEriRec * slot;
    const double h = r[9], Pw = r[10];
    if (r[11] == 0.0) {                 // a dead (zero-weight) entry
        J[a] = 0.0;
        for (int c = 0; c < 20; ++c) contrib[(int64_t)c * n + a] = 0.0;
        return;
    }
    double m[kEriAcc];
    for (int c = 0; c < kEriAcc; ++c) {
        double s = 0.0;
        for (int64_t k = 0; k < slabs; ++k) s += partial[(k * kEriAcc + c) * n + slot];
        m[c] = s;
    }
    J[a] = h * kPrefEri * m[0];
    const double gh = Pw * kPrefEri * m[0];
    const double sc = Pw * h * kPrefEri;
    const double Ai[6] = {r[0], r[1], r[2], r[3], r[4], r[5]};
    const double GT[6] = {sc * m[1], sc * m[2], sc * m[3], sc * m[4], sc * m[5], sc * m[6]};
    double gP[3] = {sc * m[7], sc * m[8], sc * m[9]};
    // dE/dA = -A^-1 GT A^-1 - gh h A^-1 / 2
    double X[9];
    sym_mul(Ai, GT, X);
    const double ai[9] = {Ai[0], Ai[3], Ai[4], Ai[3], Ai[1], Ai[5], Ai[4], Ai[5], Ai[2]};
    const int rr_[6] = {0, 1, 2, 0, 0, 1}, cc_[6] = {0, 1, 2, 1, 2, 2};
    double Gh[6];
    for (int k = 0; k < 6; ++k) {
        const int rw = rr_[k], cl = cc_[k];
        const double xa = X[3 * rw] * ai[cl] + X[3 * rw + 1] * ai[3 + cl] + X[3 * rw + 2] * ai[6 + cl];
        Gh[k] = -xa - 0.5 * gh * h * Ai[k];
    }
    const int64_t i = pi[a], j = pj[a];
    // h = KN det(A)^(-1/2): dE/dKN = gh det(A)^(-1/2) = gh h / KN (KN > 0 for every listed pair)
    const double Ni = Nrm[i], Nj = Nrm[j];
    const Sym3 Asi = load_sym(A6 + 6 * i), Asj = load_sym(A6 + 6 * j);
    const double mui[3] = {mu[3 * i], mu[3 * i + 1], mu[3 * i + 2]};
    const double muj[3] = {mu[3 * j], mu[3 * j + 1], mu[3 * j + 2]};
    Sym3 Ahp;
    double Pc[3], KN;
    pair_quantities(Asi, Asj, mui, muj, Ni, Nj, &Ahp, Pc, &KN);
    const double gKN = gh * sqrt(1.0 / det3(Ahp));
    pair_reverse(n, a, i, j, A6, mu, Nrm, Gh, gP, gKN, contrib);
}

// ------------------------------------------------------------------ exchange three-centre block
// Bt[perm[slot] * ldb + l] = (P|a) for the aux function of slot q0 + l (l < W) and the pair group
// of each slot (the list entries of one unordered splat pair share one product Gaussian, so one
// row serves them all), the record carrying q_a = w_a: the screened block of RI-K
// (gs_dft/coulomb/ri.py:527-531, full_isobra_block), written rather than contracted. One lane per
// slot (the pair order of the reverse, so the 64 pairs of a wave are close in space and width
// and the node screen fires for whole waves) and the aux records
// of slots q0 + l wave-uniform and centre-grouped (d, A d, q0..q2 formed once per centre, x[3] =
// KN_P): block (x, y) covers the pair slots [256 x, 256 x + 256) and the sixteen aux slots from
// 16 y on; each lane's sixteen values go through LDS and are written as one row segment
// Bt[perm[slot] * ldb + 16 y ...] (16-byte stores when kPair: ldb even, Bt 16-byte aligned).
constexpr int kBlockRecs = 16;

template <bool kPair, int kN>
__global__ __launch_bounds__(256) void k_exch_block_pairs(int64_t n,
                                                          const double* __restrict__ rec,
                                                          const int32_t* __restrict__ perm,
                                                          int64_t W, const double* __restrict__ aux,
                                                          int64_t ldb, double* __restrict__ Bt,
                                                          unsigned long long* __restrict__ work,
                                                          const int64_t* __restrict__ n_live) {
    // whole workgroups past the real slots leave at once (workgroup-uniform, before any barrier)
    if (n_live && (int64_t)blockIdx.x * blockDim.x >= *n_live) return;
    __shared__ double tab[256];
    __shared__ double val[kBlockRecs][256];
    for (int i = threadIdx.x; i < 256; i += blockDim.x) tab[i] = exp2_frac_lead(i);
    __syncthreads();
    const int64_t slot = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    const bool live = slot < (n_live ? *n_live : n);   // n_live: a device count of real slots
    const double* __restrict__ r = rec + kRec * (live ? slot : 0);
    const double I1 = r[0], I2 = r[1], I3 = r[2];
    const double xx = r[3], yy = r[4], zz = r[5], xy = r[6], xz = r[7], yz = r[8];
    const double Px = live ? r[9] : kFarAway, Py = live ? r[10] : kFarAway,
                 Pz = live ? r[11] : kFarAway;
    const double coef = r[12];
    const int64_t l0 = (int64_t)blockIdx.y * kBlockRecs;
    const int nrec = (int)min((int64_t)kBlockRecs, W - l0);
    double q0d = 0, q1 = 0, X0 = 0, rr = 0, cf = coef;
    uint32_t nodes = 0;
    for (int j = 0; j < nrec; ++j) {
        const double* __restrict__ x = aux + kAuxRec * (l0 + j);
        if (j == 0 || new_centre(x)) {           // wave-uniform
            const double dx = x[0] - Px, dy = x[1] - Py, dz = x[2] - Pz;
            const double ax = xx * dx + xy * dy + xz * dz;
            const double ay = xy * dx + yy * dy + yz * dz;
            const double az = xz * dx + yz * dy + zz * dz;
            q0d = dx * dx + dy * dy + dz * dz;
            q1 = dx * ax + dy * ay + dz * az;
            const double q2 = ax * ax + ay * ay + az * az;
            X0 = I3 * q0d;
            rr = I1 * q1 - q2;
            cf = (q0d == q0d) ? coef : q0d;          // a NaN centre propagates
        }
        double F = 0.0;
        // each node's constants are read one node ahead, so their scalar load overlaps the
        // previous node's arithmetic
        double n_s = x[rec_s(0)], n_wh = x[rec_wh(0)], n_is = x[rec_is(0)];
        auto node = [&](auto tc) {
            constexpr int t = decltype(tc)::value;
            const double st = n_s, wh = n_wh, is = n_is;
            if constexpr (t + 1 < kN) {
                n_s = x[rec_s(t + 1)];
                n_wh = x[rec_wh(t + 1)];
                n_is = x[rec_is(t + 1)];
            }
            const double Pr = __builtin_fma(is, I3, __builtin_fma(st, I1 + st, I2));
            const double Qn = __builtin_fma(st, __builtin_fma(st, q1, rr), X0);
            const NodeArgH v = node_arg_h(Pr, Qn);
            F = __builtin_fma(wh * v.y0, exp_neg_tab_k(v.arg, tab), F);
            // keep the next node's loads ahead of the early exit (not sunk past it)
            if constexpr (t + 1 < kN) asm volatile("" ::"s"(n_s), "s"(n_wh), "s"(n_is));
            return screen_after<kN>(t) && wave_all_beyond_h(v.arg);
        };
        nodes += node_loop<0, kN>(node);
        val[j][threadIdx.x] = (F * cf) * x[3];
    }
    count_work(work, live, nodes);
    if (!live) return;
    double* row = Bt + (int64_t)perm[slot] * ldb + l0;
    if (kPair && nrec == kBlockRecs) {
#pragma unroll
        for (int j = 0; j < kBlockRecs; j += 2)
            *reinterpret_cast<double2*>(row + j) = make_double2(val[j][threadIdx.x],
                                                                val[j + 1][threadIdx.x]);
    } else {
        for (int j = 0; j < nrec; ++j) row[j] = val[j][threadIdx.x];
    }
}

// acc[c][slot] = (first ? 0 : acc[c][slot]) + sum over slabs of partial[slab][c][slot].
__global__ void k_acc_fold(int64_t n, int64_t slabs, const double* __restrict__ partial,
                           double* __restrict__ acc, int first) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t >= n * kAcc) return;
    const int64_t c = t / n, slot = t % n;
    double v = first ? 0.0 : acc[t];
    for (int64_t k = 0; k < slabs; ++k) v += partial[(k * kAcc + c) * n + slot];
    acc[t] = v;
}

// buf[0][c][slot] += buf[1][c][slot] + ... + buf[slabs - 1][c][slot], in slab order (the running
// moment sums of the DF-J reverse and the later slabs of one launch, stride kAcc n per slab).
__global__ void k_slab_fold(int64_t n, int64_t slabs, double* __restrict__ buf) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t >= n * kAcc) return;
    double v = buf[t];
    for (int64_t k = 1; k < slabs; ++k) v += buf[k * kAcc * n + t];
    buf[t] = v;
}

// inv[perm[slot]] = slot.
__global__ void k_inv_perm(int64_t n, const int32_t* __restrict__ perm, int32_t* __restrict__ inv) {
    const int64_t slot = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (slot < n) inv[perm[slot]] = (int32_t)slot;
}

// ------------------------------------------------------------------ work split

struct Split {
    int64_t slabs;
    int64_t per_slab;
};

Split bwd_split(int64_t N, int64_t n) {
    const int64_t groups = n > 0 ? (n + 255) / 256 : 1;
    const int64_t target = 256 * 4 * 4;
    int64_t slabs = (target + groups - 1) / groups;
    slabs = slabs < 1 ? 1 : slabs;
    const int64_t max_slabs = (N + 15) / 16;
    if (slabs > max_slabs) slabs = max_slabs < 1 ? 1 : max_slabs;
    if (slabs > 65535) slabs = 65535;
    const int64_t per = (N + slabs - 1) / slabs;
    return Split{(N + per - 1) / (per > 0 ? per : 1), per > 0 ? per : 1};
}

// The DF-J reverse: besides enough slabs to fill the device (bwd_split), the aux records are cut
// into slabs of at most kL2Records records (2.9 MB) so that the workgroups running together walk
// one slab, which then stays in the XCD's 4 MB L2 instead of coming from the MALL once per
// workgroup: at globule700 (80,000 records, 11.2 M pairs) 20 slabs, and the reverse takes 8.49
// instead of 9.05 s. The result depends on the split only through the order in which the slabs'
// moments are added (fixed for given N and n).
constexpr int64_t kL2Records = 4096;
constexpr double kSlabBudget = 5.0 * (1ull << 30);

Split bwd_split_records(int64_t N, int64_t n) {
    Split sp = bwd_split(N, n);
    const int64_t want = (N + kL2Records - 1) / kL2Records;
    if (N <= 0 || sp.slabs >= want) return sp;
    int64_t slabs = want > 65535 ? 65535 : want;
    const int64_t per = (N + slabs - 1) / slabs;
    return Split{(N + per - 1) / per, per};
}

// Slabs per launch of the DF-J reverse: every slab in one launch while their partial moments
// (kAcc n doubles each) fit in kSlabBudget, else launches of `per_launch` slabs one after the
// other, each adding its slabs' moments to running sums (the first slab in the kernel, the rest by
// k_slab_fold), so the moment storage is per_launch slabs whatever the slab count: 4.5 GB at
// 11.2 M pairs (2 slabs a launch), 4.1 GB at 20.6 M (1). The sums run in slab order either way,
// so the result does not depend on the launch grouping.
int64_t bwd_slabs_per_launch(int64_t N, int64_t n) {
    const Split sp = bwd_split_records(N, n);
    const double per_slab_bytes = 8.0 * kAcc * (double)(n > 0 ? n : 1);
    int64_t r = (int64_t)(kSlabBudget / per_slab_bytes);
    if (r < 1) r = 1;
    return r < sp.slabs ? r : sp.slabs;
}

struct GammaWs {
    double *A6, *Nrm, *beta, *kn, *q, *rec, *partial;
    double *aux, *acc, *contrib, *rec_sorted;
    PairOrderWs pair_order;
};

int layout_gamma(Arena& ar, int64_t M, int64_t N, int64_t n, bool reverse, GammaWs* w) {
    w->A6 = ar.take<double>(6 * M + 1);
    w->Nrm = ar.take<double>(M + 1);
    w->beta = ar.take<double>(N + 1);
    w->kn = ar.take<double>(N + 1);
    w->q = ar.take<double>(n + 1);
    w->partial = w->aux = w->acc = w->contrib = w->rec_sorted = w->rec = nullptr;
    if (!reverse) {
        w->rec = ar.take<double>(kRec * n + kRec);
        const int64_t groups = n > 0 ? (n + kFwdPairs - 1) / kFwdPairs : 1;
        w->aux = ar.take<double>(kAuxRec * N + kAuxRec);
        w->rec_sorted = ar.take<double>(kRec * n + kRec);
        GSDFT_TRY(pair_order_layout(ar, n, &w->pair_order));
        w->partial = ar.take<double>(groups * N + 1);
    } else {
        // at least as many slabs as bwd_split's, which the nuclear pass launches with; the
        // unsorted pair records are dead once gathered into slot order, before any moment is
        // written, so they occupy the start of the moment storage
        const int64_t slabs = std::max(bwd_split(N, n).slabs, bwd_slabs_per_launch(N, n));
        w->aux = ar.take<double>(kAuxRec * N + kAuxRec);
        w->acc = ar.take<double>(std::max(slabs * kAcc * n + 1, kRec * n + kRec));
        w->rec = w->acc;
        w->rec_sorted = ar.take<double>(kRec * n + kRec);
        GSDFT_TRY(pair_order_layout(ar, n, &w->pair_order));
        w->contrib = ar.take<double>(20 * n + 1);
    }
    return GSDFT_OK;
}

int launch_pair_density(int64_t n, const int32_t* pi, const int32_t* pj, const double* weight,
                        int64_t k, const double* C, const double* occ, double* q, hipStream_t s) {
    if (n <= 0) return GSDFT_OK;
    // one pass while G n work-items fit a grid dimension, else the grid strides over the pairs
    auto grid = [n](int G) {
        return (unsigned)std::min<int64_t>((n * G + 255) / 256, (int64_t)(UINT32_MAX / 256));
    };
    if (k <= 8) {
        k_pair_density<8><<<grid(8), 256, 0, s>>>(n, pi, pj, weight, k, C, occ, q);
    } else if (k <= 16) {
        k_pair_density<16><<<grid(16), 256, 0, s>>>(n, pi, pj, weight, k, C, occ, q);
    } else if (k <= 32) {
        k_pair_density<32><<<grid(32), 256, 0, s>>>(n, pi, pj, weight, k, C, occ, q);
    } else if (k <= 64 * 32) {
        // one wave per run of kDensityRun pairs (at most n / 16 waves: within one grid dimension
        // for any list the entry points accept)
        const unsigned blocks = (unsigned)(((n + kDensityRun - 1) / kDensityRun + 3) / 4);
        if (k <= 64 * 8)
            k_pair_density_run<8><<<blocks, 256, 0, s>>>(n, pi, pj, weight, k, C, occ, q);
        else if (k <= 64 * 16)
            k_pair_density_run<16><<<blocks, 256, 0, s>>>(n, pi, pj, weight, k, C, occ, q);
        else if (k <= 64 * 24)
            k_pair_density_run<24><<<blocks, 256, 0, s>>>(n, pi, pj, weight, k, C, occ, q);
        else
            k_pair_density_run<32><<<blocks, 256, 0, s>>>(n, pi, pj, weight, k, C, occ, q);
    } else {
        k_pair_density<64><<<grid(64), 256, 0, s>>>(n, pi, pj, weight, k, C, occ, q);
    }
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}

int launch_dC(int64_t M, int64_t k, const int32_t* row_ptr, const int32_t* row_perm,
              const int32_t* col_ptr, const int32_t* col_perm, const int32_t* pi,
              const int32_t* pj, const double* J, const double* weight, const double* C,
              const double* occ, double* dC, hipStream_t s) {
    constexpr int kCH = 1;                                 // orbitals per thread and chunk
    const int64_t nchunks = (k + 256 * kCH - 1) / (256 * kCH);
    if (M * nchunks > (int64_t)(UINT32_MAX / 256))
        return fail(GSDFT_ERR_ARG, "dC: M = %lld x %lld orbital chunks too many for one launch",
                    (long long)M, (long long)nchunks);
    k_dC<kCH><<<xcd_grid(M * nchunks), 256, 0, s>>>(M, k, nchunks, row_ptr, row_perm, col_ptr,
                                                    col_perm, pi, pj, J, weight, C, occ, dC);
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}

// Shared prologue of forward and reverse: chart, aux quantities (skipped for a null log_alpha),
// pair density (zero for a null C), pair records.
int gamma_prologue(int64_t M, const double* quat, const double* log_scale, const double* centers,
                   int64_t k, const double* C, const double* occ, int64_t N,
                   const double* log_alpha, int64_t n, const int32_t* pi, const int32_t* pj,
                   const double* weight, GammaWs& w, hipStream_t s) {
    GSDFT_TRY(launch_chart(M, quat, log_scale, w.A6, w.Nrm, s));
    if (log_alpha) {
        k_aux_prep<<<blocks_for(N, 256), 256, 0, s>>>(N, log_alpha, w.beta, w.kn);
        GSDFT_HIP(hipGetLastError());
    }
    if (n > 0) {
        if (C) {
            GSDFT_TRY(launch_pair_density(n, pi, pj, weight, k, C, occ, w.q, s));
        } else {                                 // values only: q = 0 zeroes every gradient term
            k_fill<<<blocks_for(n, 256), 256, 0, s>>>(n, 0.0, w.q);
            GSDFT_HIP(hipGetLastError());
        }
        k_pair_rec<<<blocks_for(n, 256), 256, 0, s>>>(n, pi, pj, w.A6, centers, w.Nrm, w.q, w.rec);
        GSDFT_HIP(hipGetLastError());
    }
    return GSDFT_OK;
}


}  // namespace


// ------------------------------------------------------------------ exchange: three-centre passes

// out[g] = rec[perm[g]] for g < *n_live (records past it are left alone).
__global__ void k_rec_gather_live(int64_t n, const int64_t* __restrict__ n_live,
                                  const int32_t* __restrict__ perm, const double* __restrict__ rec,
                                  double* __restrict__ out) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t >= n * kRec || t / kRec >= *n_live) return;
    out[t] = rec[(int64_t)perm[t / kRec] * kRec + t % kRec];
}

// slot_pair[slot] = rep[perm[slot]] (slots past the groups get whatever rep holds there: unused).
__global__ void k_compose(int64_t n, const int32_t* __restrict__ perm,
                          const int32_t* __restrict__ rep, int32_t* __restrict__ out) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (t < n) out[t] = rep[perm[t]];
}

int exch_tc_layout(Arena& ar, int64_t M, int64_t N, int64_t n, int64_t Pc, bool grads,
                   ExchTcWs* w) {
    *w = ExchTcWs{};
    w->A6 = ar.take<double>(6 * M + 1);
    w->Nrm = ar.take<double>(M + 1);
    w->beta = ar.take<double>(N + 1);
    w->kn = ar.take<double>(N + 1);
    w->q = ar.take<double>(n + 1);
    w->rec = ar.take<double>(kRec * n + kRec);
    w->rec_grp = ar.take<double>(kRec * n + kRec);
    w->rec_sorted = ar.take<double>(kRec * n + kRec);
    w->aux = ar.take<double>(kAuxRec * N + kAuxRec);
    w->ent_group = ar.take<int32_t>(n + 1);
    w->ent_pos = ar.take<int32_t>(n + 1);
    w->grp_first = ar.take<int32_t>(n + 2);
    w->grp_rep = ar.take<int32_t>(n + 1);
    w->slot_pair = ar.take<int32_t>(n + 1);
    w->head = ar.take<int32_t>(n + 1);
    w->n_groups_dev = ar.take<int64_t>(1);
    w->scan_bytes = pair_groups_scan_bytes(n);
    w->scan_tmp = ar.take<char>(w->scan_bytes + 1);
    GSDFT_TRY(pair_order_layout(ar, n, &w->pair_order));
    if (grads) {
        // bwd_split(W, m).slabs x n (the moments' slot stride is n) over every chunk width
        // W <= Pc and slab estimate m >= n / 2: at most (4096 / ceil(m / 256) + 1) n <=
        // 2 x 4096 x 256 + n + 512, and at most the slab cap x n
        int64_t cap = std::min<int64_t>((Pc + 15) / 16, 65535);
        if (cap < 1) cap = 1;
        const int64_t bound = std::min<int64_t>(cap * n, 2 * 4096 * 256 + n + 512);
        w->part = ar.take<double>(kAcc * bound + 1);
        w->acc = ar.take<double>(kAcc * n + 1);
        w->J = ar.take<double>(n + 1);
        w->contrib = ar.take<double>(20 * n + 1);
    }
    return GSDFT_OK;
}

int exch_tc_prologue(int64_t M, const double* quat, const double* log_scale,
                     const double* centers, int64_t N, const double* log_alpha,
                     const double* aux_centers, int64_t n, const int32_t* pi, const int32_t* pj,
                     const double* weight, bool grads, const ExchTcWs& w, hipStream_t s) {
    (void)grads;
    GSDFT_TRY(launch_chart(M, quat, log_scale, w.A6, w.Nrm, s));
    k_aux_prep<<<blocks_for(N, 256), 256, 0, s>>>(N, log_alpha, w.beta, w.kn);
    GSDFT_HIP(hipGetLastError());
    if (n <= 0) return GSDFT_OK;
    if (weight) {
        GSDFT_HIP(hipMemcpyAsync(w.q, weight, n * sizeof(double), hipMemcpyDeviceToDevice, s));
    } else {
        k_fill<<<blocks_for(n, 256), 256, 0, s>>>(n, 1.0, w.q);
        GSDFT_HIP(hipGetLastError());
    }
    k_pair_rec<<<blocks_for(n, 256), 256, 0, s>>>(n, pi, pj, w.A6, centers, w.Nrm, w.q, w.rec);
    GSDFT_HIP(hipGetLastError());
    const int64_t G = (N % M == 0) ? N / M : 1;
    k_aux_bwd_prep<<<blocks_for(N, 256), 256, 0, s>>>(N, G, w.beta, w.kn, aux_centers, nullptr,
                                                      nullptr, kAuxPlain, w.table, w.aux);
    GSDFT_HIP(hipGetLastError());
    // one record per group (its first entry's), then the groups' slot order: the group count
    // stays on the device, the first n_groups_dev slots are the groups and the rest idle
    GSDFT_TRY(launch_pair_groups(M, n, pi, pj, w.q, w.pair_order, w.head, w.scan_tmp,
                                 w.scan_bytes, w.ent_group, w.ent_pos, w.grp_first, w.grp_rep,
                                 w.n_groups_dev, s));
    k_rec_gather_live<<<blocks_for(n * kRec, 256), 256, 0, s>>>(n, w.n_groups_dev, w.grp_rep,
                                                                 w.rec, w.rec_grp);
    GSDFT_HIP(hipGetLastError());
    GSDFT_TRY(launch_pair_order(n, w.rec_grp, kRec, w.pair_order, s, w.n_groups_dev));
    k_rec_gather_live<<<blocks_for(n * kRec, 256), 256, 0, s>>>(n, w.n_groups_dev,
                                                                 w.pair_order.perm, w.rec_grp,
                                                                 w.rec_sorted);
    k_compose<<<blocks_for(n, 256), 256, 0, s>>>(n, w.pair_order.perm, w.grp_rep, w.slot_pair);
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}

int exch_tc_block(int64_t M, int64_t N, int64_t q0, int64_t W, const double* aux_centers,
                  int64_t n, int64_t ldb, double* Bt, const ExchTcWs& w, hipStream_t s) {
    if (n <= 0 || W <= 0) return GSDFT_OK;
    (void)M; (void)N; (void)aux_centers;
    const int64_t gy = (W + kBlockRecs - 1) / kBlockRecs;
    if (gy > 65535) return fail(GSDFT_ERR_ARG, "exchange: aux chunk too wide");
    dim3 grid((unsigned)((n + 255) / 256), (unsigned)gy);
    const bool pair = ldb % 2 == 0 && reinterpret_cast<uintptr_t>(Bt) % 16 == 0;
    profile_begin(kProfExchBlock, s);
    unsigned long long* work = profile_work_counter(kProfExchBlock);
    const double* aux = w.aux + kAuxRec * q0;
    if (w.table.n == kLrNodes) {
        if (pair)
            k_exch_block_pairs<true, kLrNodes><<<grid, 256, 0, s>>>(n, w.rec_sorted,
                                                                    w.pair_order.perm, W, aux, ldb,
                                                                    Bt, work, w.n_groups_dev);
        else
            k_exch_block_pairs<false, kLrNodes><<<grid, 256, 0, s>>>(n, w.rec_sorted,
                                                                     w.pair_order.perm, W, aux,
                                                                     ldb, Bt, work, w.n_groups_dev);
    } else {
        if (pair)
            k_exch_block_pairs<true, kNodes><<<grid, 256, 0, s>>>(n, w.rec_sorted,
                                                                  w.pair_order.perm, W, aux, ldb,
                                                                  Bt, work, w.n_groups_dev);
        else
            k_exch_block_pairs<false, kNodes><<<grid, 256, 0, s>>>(n, w.rec_sorted,
                                                                   w.pair_order.perm, W, aux, ldb,
                                                                   Bt, work, w.n_groups_dev);
    }
    profile_end(kProfExchBlock, s);
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}

int exch_tc_reverse(int64_t N, int64_t q0, int64_t W, int64_t n, int64_t n_est,
                    const double* Tbar, int64_t ldt, bool group_rows, bool first,
                    const ExchTcWs& w, hipStream_t s) {
    if (n <= 0 || W <= 0) return GSDFT_OK;
    const Split sp = bwd_split(W, std::max<int64_t>(1, std::min(n, n_est)));
    dim3 grid((unsigned)((n + 255) / 256), (unsigned)sp.slabs);
    profile_begin(kProfExchBwd, s);
    if (w.table.n == kLrNodes)
        k_gamma_bwd<true, false, false, kLrNodes><<<grid, 256, 0, s>>>(
            n, w.rec_sorted, W, w.aux + kAuxRec * q0, sp.per_slab, w.part,
            profile_work_counter(kProfExchBwd), Tbar, ldt, nullptr, w.pair_order.perm,
            w.grp_first, w.n_groups_dev, group_rows ? 1 : 0);
    else
        k_gamma_bwd<true><<<grid, 256, 0, s>>>(n, w.rec_sorted, W, w.aux + kAuxRec * q0,
                                               sp.per_slab, w.part,
                                               profile_work_counter(kProfExchBwd), Tbar, ldt,
                                               nullptr, w.pair_order.perm, w.grp_first,
                                               w.n_groups_dev, group_rows ? 1 : 0);
    profile_end(kProfExchBwd, s);
    GSDFT_HIP(hipGetLastError());
    k_acc_fold<<<blocks_for(n * kAcc, 256), 256, 0, s>>>(n, sp.slabs, w.part, w.acc, first ? 1 : 0);
    GSDFT_HIP(hipGetLastError());
    (void)N;
    return GSDFT_OK;
}

int exch_tc_finish(int64_t M, int64_t n, const int32_t* pi, const int32_t* pj,
                   const double* weight, const double* quat, const double* log_scale,
                   const double* centers, const int32_t* row_ptr, const int32_t* row_perm,
                   const int32_t* col_ptr, const int32_t* col_perm, double* dquat,
                   double* dlog_scale, double* dcenters, const ExchTcWs& w, hipStream_t s) {
    if (n > 0) {
        // every entry but its group's first contributes nothing of its own
        k_fill<<<blocks_for(20 * n, 256), 256, 0, s>>>(20 * n, 0.0, w.contrib);
        k_fill<<<blocks_for(n, 256), 256, 0, s>>>(n, 0.0, w.J);
        GSDFT_HIP(hipGetLastError());
        k_pair_finalize<<<blocks_for(n, 256), 256, 0, s>>>(
            n, n, 1, kPref3c, w.slot_pair, pi, pj, weight, w.A6, centers, w.Nrm, w.rec_sorted,
            w.acc, w.J, w.contrib, w.n_groups_dev);
        GSDFT_HIP(hipGetLastError());
    }
    k_splat_grad<<<blocks_for(M * 64, 256), 256, 0, s>>>(M, n, row_ptr, row_perm, col_ptr,
                                                         col_perm, w.contrib, quat, log_scale,
                                                         dquat, dlog_scale, dcenters);
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}

}  // namespace gsdft

using namespace gsdft;

static Scales scale_chunk(const double* scales, int n_scales, int s0) {
    Scales sc{};
    sc.s0 = s0;
    sc.n = std::min(16, n_scales - s0);
    for (int i = 0; i < sc.n; ++i) sc.v[i] = scales[s0 + i];
    return sc;
}

extern "C" int gsdft_product_aux(int64_t M, const double* quat, const double* log_scale,
                                 const double* centers, const double* scales, int n_scales,
                                 double* log_alpha, double* aux_centers, void* workspace,
                                 size_t workspace_bytes, void* stream) {
    (void)workspace;
    (void)workspace_bytes;
    if (M <= 0 || n_scales <= 0 || !scales || !quat || !log_scale || !centers || !log_alpha ||
        !aux_centers)
        return fail(GSDFT_ERR_ARG, "gsdft_product_aux: need M > 0, at least one scale and every "
                    "array");
    hipStream_t s = (hipStream_t)stream;
    for (int s0 = 0; s0 < n_scales; s0 += 16) {
        k_product_aux<<<blocks_for(M, 256), 256, 0, s>>>(M, quat, log_scale, centers,
                                                          scale_chunk(scales, n_scales, s0),
                                                          log_alpha, aux_centers);
        GSDFT_HIP(hipGetLastError());
    }
    return GSDFT_OK;
}

extern "C" int gsdft_product_aux_pairs(int64_t M, const double* quat, const double* log_scale,
                                       const double* centers, int64_t n, const int32_t* pi,
                                       const int32_t* pj, const double* valid,
                                       const double* scales, int n_scales, double* log_alpha,
                                       double* aux_centers, void* workspace,
                                       size_t workspace_bytes, void* stream) {
    if (M <= 0 || n < 0 || n_scales <= 0 || !scales || !quat || !log_scale || !centers ||
        (n > 0 && (!pi || !pj || !log_alpha || !aux_centers)))
        return fail(GSDFT_ERR_ARG, "gsdft_product_aux_pairs: need M > 0, n >= 0, at least one "
                    "scale and every array");
    GSDFT_TRY(check_pairs(n, "gsdft_product_aux_pairs"));
    if (n == 0) return GSDFT_OK;
    hipStream_t s = (hipStream_t)stream;
    Arena ar{(char*)workspace, workspace_bytes, 0};
    double* A6 = ar.take<double>(6 * M + 1);
    double* Nrm = ar.take<double>(M + 1);
    if (!A6 || !Nrm) return fail(GSDFT_ERR_WORKSPACE, "gsdft_product_aux_pairs: workspace too small");
    GSDFT_TRY(launch_chart(M, quat, log_scale, A6, Nrm, s));
    for (int s0 = 0; s0 < n_scales; s0 += 16) {
        k_product_aux_pairs<<<blocks_for(n, 256), 256, 0, s>>>(
            n, pi, pj, valid, A6, Nrm, centers, scale_chunk(scales, n_scales, s0), log_alpha,
            aux_centers);
        GSDFT_HIP(hipGetLastError());
    }
    return GSDFT_OK;
}

// Blocked Cholesky: panels of kCholNb rows.
constexpr int64_t kCholNb = 2048;

extern "C" int gsdft_metric_workspace_size(int64_t N, size_t* bytes) {
    if (N < 0 || !bytes) return fail(GSDFT_ERR_ARG, "metric_workspace_size: bad arguments");
    Arena ar{nullptr, 0, 0};
    ar.take<double>(2 * N + 2);
    ar.take<int64_t>(2);
    *bytes = ar.need();
    return GSDFT_OK;
}

extern "C" int gsdft_aux_metric(int64_t N, const double* log_alpha, const double* aux_centers,
                                double lam, double omega, double* V, void* workspace,
                                size_t workspace_bytes, void* stream) {
    if (N <= 0 || !log_alpha || !aux_centers || !V)
        return fail(GSDFT_ERR_ARG, "gsdft_aux_metric: bad arguments");
    if (!(omega >= 0.0) || std::isinf(omega))
        return fail(GSDFT_ERR_ARG, "gsdft_aux_metric: omega must be finite and >= 0");
    if ((N + 3) / 4 > 65535) return fail(GSDFT_ERR_ARG, "gsdft_aux_metric: N too large");
    hipStream_t s = (hipStream_t)stream;
    Arena ar{(char*)workspace, workspace_bytes, 0};
    double* bk = ar.take<double>(2 * N + 2);
    if (!bk) return fail(GSDFT_ERR_WORKSPACE, "gsdft_aux_metric: workspace too small");
    k_aux_prep<<<blocks_for(N, 256), 256, 0, s>>>(N, log_alpha, bk, bk + N);
    dim3 grid((unsigned)((N + 63) / 64), (unsigned)((N + 4 * kMetricRows - 1) / (4 * kMetricRows)));
    profile_begin(kProfMetric, s);
    k_metric<false><<<grid, 256, 0, s>>>(N, bk, bk + N, aux_centers, lam, omega, V);
    profile_end(kProfMetric, s);
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}

constexpr int kPanelRows = 128;     // rows per diagonal block (inner factorisation, panel solve)
constexpr int kPotfThreads = 1024;

__global__ void k_info_reset(int64_t* __restrict__ info) { *info = 0; }

// Unblocked upper Cholesky of one ib x ib diagonal block (ib <= 128; column-major, leading
// dimension N, A(r, c) at A[c N + r] for r <= c), in place. Step j subtracts
// A(j, r) A(j, c) / A(j, j) from A(r, c) for j < r <= c; the rows are scaled at the end:
// U(j, j) = sqrt(A(j, j)), U(j, c) = A(j, c) / U(j, j). A pivot that is not positive records
// base + j + 1 in *info unless an earlier minor has failed (the factor is then meaningless, as
// with any failed factorisation).
// Thread t holds column c = t % 128 in registers: during block J of eight steps, v[i] is row
// rg + 8 (J + i) of the row group rg = t / 128 (wave-uniform); at the end of the block v[0] is
// final, goes to LDS, and the registers shift down. Step j reads row j from LDS, where the threads
// holding it published it at the end of step j - 1 (it is final then), in one of two buffers, so
// each step takes one barrier. The published row keeps A(j, c) at (c % 8) 16 + c / 8, so a
// thread's 16 rows are 16 consecutive entries: all are read at once, unconditionally, and the
// registers past the thread's last row take updates that are never stored (their reads land on
// the next row group's entries or on the zero padding past the row).
// Every FMA of a stored entry is the one the right-looking order applies, in the same order, so
// the factor does not depend on the thread layout. Steps past ib run on the zero padding: they
// touch only columns >= ib, which are never stored or read. The block is staged through LDS so the
// global loads and stores stay coalesced.
__global__ __launch_bounds__(kPotfThreads) void k_potf2(int64_t N, double* __restrict__ A, int ib,
                                                        int64_t base,
                                                        int64_t* __restrict__ info) {
    constexpr int kLoads = kPanelRows * kPanelRows / kPotfThreads;  // rows per thread (16)
    constexpr int kGroups = kPotfThreads / kPanelRows;              // row groups (8)
    static_assert(kLoads * kGroups == kPanelRows, "one register per row of the thread's group");
    constexpr int kRowPad = kPanelRows + kLoads;
    __shared__ double As[kPanelRows][kPanelRows + 1];
    __shared__ double rowj[2][kRowPad];
    __shared__ double sq[kPanelRows];
    const int t = threadIdx.x;
    {
        double w[kLoads];
#pragma unroll
        for (int q = 0; q < kLoads; ++q) {
            const int e = t + q * kPotfThreads, c = e >> 7, r = e & (kPanelRows - 1);
            w[q] = (c < ib && r <= c) ? A[c * N + r] : 0.0;
        }
#pragma unroll
        for (int q = 0; q < kLoads; ++q) {
            const int e = t + q * kPotfThreads;
            As[e >> 7][e & (kPanelRows - 1)] = w[q];
        }
    }
    if (t < 2 * kLoads) rowj[t / kLoads][kPanelRows + t % kLoads] = 0.0;
    __syncthreads();
    const int c = t & (kPanelRows - 1);
    const int pc = (c % kGroups) * kLoads + c / kGroups;          // c's place in a published row
    const int rg = __builtin_amdgcn_readfirstlane(t >> 7);
    double v[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) v[i] = As[c][rg + kGroups * i];
    if (t < kPanelRows) rowj[0][pc] = As[c][0];
    __syncthreads();
    int bad = 0;                                  // thread 0: first failing step + 1
    for (int j = 0; j < kPanelRows; ++j) {
        const int J = j / kGroups, jj = j % kGroups;
        const double* __restrict__ rw = rowj[j & 1];
        const double piv = rw[jj * kLoads + J];
        if (t == 0 && j < ib && !(piv > 0.0) && bad == 0) bad = j + 1;
        if (c > j) {
            const double uc = rw[pc] / piv;
            const double* __restrict__ rr = rw + rg * kLoads + J;   // rows rg + 8 (J + i)
            double a[kLoads];
#pragma unroll
            for (int i = 0; i < kLoads; ++i) a[i] = rr[i];
            if (rg > jj) v[0] = __builtin_fma(-a[0], uc, v[0]);    // rows j < r only
#pragma unroll
            for (int i = 1; i < kLoads; ++i) v[i] = __builtin_fma(-a[i], uc, v[i]);
        }
        if (jj == kGroups - 1) {                  // row rg + 8 J is final
            As[c][rg + kGroups * J] = v[0];
#pragma unroll
            for (int i = 0; i + 1 < kLoads; ++i) v[i] = v[i + 1];
            v[kLoads - 1] = 0.0;
        }
        // publish row j + 1 (in v[0] of row group (j + 1) % 8)
        if (j + 1 < kPanelRows && rg == (j + 1) % kGroups) rowj[(j + 1) & 1][pc] = v[0];
        __syncthreads();
    }
    if (t < ib) sq[t] = sqrt(As[t][t]);
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kLoads; ++q) {
        const int e = t + q * kPotfThreads, cc = e >> 7, r = e & (kPanelRows - 1);
        if (cc < ib && r <= cc) A[cc * N + r] = r == cc ? sq[r] : As[cc][r] / sq[r];
    }
    if (t == 0 && bad != 0 && *info == 0) *info = base + bad;
}

// X <- U^-T X for one diagonal block on the FP64 MFMA: U is ib x ib upper (column-major, leading
// dimension N; U(c, r) at U[r N + c]), X is ib x T (column-major, leading dimension ldx). Each wave
// holds 16 columns of X as eight 16 x 16 accumulator tiles, one per 16-row block
// (v_mfma_f64_16x16x4f64 layout: lane l holds rows l / 16 + 4 r, r < 4, of column l % 16). Block
// b is solved row by row on the VALU (x_i = acc * (1 / U(i, i)), broadcast from the lane group
// holding row i to all four with two permlane swaps, every row i' > i of the block takes
// -U(i, i') x_i), then every later block b' takes -U(b rows, b' columns)^T X_b in four MFMAs whose
// B operand is the solved tile's register r as it stands (row 4 r + l / 16). The MFMA adds its
// four products in order with a rounding each, so every entry gets the same FMAs in the same
// order as a row-by-row substitution. The 28 strictly-upper 16 x 16 tiles of U (negated) and the
// eight diagonal tiles (arranged so a lane reads its four rows' entries as one 32-byte run, zero
// on and below the diagonal) are staged in LDS once per workgroup, with the reciprocals of the
// diagonal. Rows past ib and columns past T are zero and not stored; every load reads an
// in-range address.
// kBack solves U X = P instead (X <- U^-1 X): the blocks and their rows from the last, row i
// subtracting U(i', i) x_i from the rows i' < i and block b subtracting U(b' rows, b columns) X_b
// from the blocks b' < b. kRowRHS takes the right-hand sides as the columns of a row-major block:
// X(r, c) at X[r ldx + c] (the solves of X U = B and X U^T = B for a column-major X).
typedef double v4d_sub __attribute__((ext_vector_type(4)));
constexpr int kSubTiles = 28;
__host__ __device__ constexpr int sub_tile(int a, int b) { return b * (b - 1) / 2 + a; }

// f(std::integral_constant<int, i>) for i = I, ..., N - 1.
template <int I, int N, class F>
__device__ __forceinline__ void static_for(F& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

// v broadcast from the 16-lane group g (compile-time) to all four groups of the wave.
template <int g>
__device__ __forceinline__ double group_bcast(double v) {
    double lo = v, hi = v;
    swap32(lo, hi);                 // lo: lanes 0-31 twice, hi: lanes 32-63 twice
    double w = g < 2 ? lo : hi;
    double e = w, o = w;
    swap16(e, o);                   // e: rows 0 and 2 of each half twice, o: rows 1 and 3
    return g % 2 == 0 ? e : o;
}

template <bool kBack, bool kRowRHS>
__global__ __launch_bounds__(256) void k_panel_subst(int64_t N, const double* __restrict__ U,
                                                     int ib, double* __restrict__ X, int64_t T,
                                                     int64_t ldx) {
    // Ut[(a, b)][k][c] = -U(16 a + k, 16 b + c) (kBack: -U(16 a + c, 16 b + k)), a < b;
    // Ud[b][i][4 g + r] = U(16 b + i, 16 b + g + 4 r) for g + 4 r > i
    // (kBack: U(16 b + g + 4 r, 16 b + i) for g + 4 r < i)
    __shared__ double Ut[kSubTiles][16][16];
    __shared__ double Ud[8][16][16];
    __shared__ double rdg[kPanelRows];
    const int t = threadIdx.x;
    const int l = t & 63, g = l >> 4;
    const int64_t cc = (int64_t)blockIdx.x * 64 + (t >> 6) * 16 + (l & 15);
    const bool live = cc < T;
    // every load reads an in-range address (columns past T and rows past ib clamped to the
    // last ones); the values that stand for nothing are zeroed. The right-hand sides and the
    // diagonal are loaded first and pinned (empty asm) before they are masked: left to itself the
    // compiler moves each right-hand-side load into a branch on its mask and waits on it there,
    // one memory round trip per value (32 in a row).
    const int64_t ccl = live ? cc : T - 1;
    auto at = [&](int row) -> int64_t { return kRowRHS ? row * ldx + ccl : ccl * ldx + row; };
    double xv[8][4];
#pragma unroll
    for (int b = 0; b < 8; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 16 * b + g + 4 * r;
            xv[b][r] = X[at(row < ib ? row : ib - 1)];
        }
    const int td = t < ib ? t : ib - 1;
    double dg = U[(int64_t)td * N + td];
#pragma unroll
    for (int b = 1; b < 8; ++b)
#pragma unroll
        for (int a = 0; a < b; ++a) {
            const int k = t & 15, c = t >> 4;
            const int row = kBack ? 16 * a + c : 16 * a + k, col = kBack ? 16 * b + k : 16 * b + c;
            const double v = U[(int64_t)min(col, ib - 1) * N + min(row, ib - 1)];
            Ut[sub_tile(a, b)][k][c] = (row < ib && col < ib) ? -v : 0.0;
        }
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const int i = t >> 4, sl = t & 15, ip = (sl >> 2) + 4 * (sl & 3);
        const int row = kBack ? 16 * b + ip : 16 * b + i, col = kBack ? 16 * b + i : 16 * b + ip;
        const double v = U[(int64_t)min(col, ib - 1) * N + min(row, ib - 1)];
        Ud[b][i][sl] = ((kBack ? ip < i : ip > i) && row < ib && col < ib) ? v : 0.0;
    }
    asm volatile("" : "+v"(dg));
    if (t < kPanelRows) rdg[t] = t < ib ? 1.0 / dg : 0.0;
    v4d_sub C[8];
#pragma unroll
    for (int b = 0; b < 8; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 16 * b + g + 4 * r;
            asm volatile("" : "+v"(xv[b][r]));
            C[b][r] = (live && row < ib) ? xv[b][r] : 0.0;
        }
    __syncthreads();
#pragma unroll
    for (int bb = 0; bb < 8; ++bb) {
        const int b = kBack ? 7 - bb : bb;
        // the block's reciprocals, lane j % 16 holding row j's (read with readlane), and each
        // step's four U entries loaded one step ahead, so the row chain waits on no LDS read
        const double rv = rdg[16 * b + (l & 15)];
        double un[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) un[r] = Ud[b][kBack ? 15 : 0][4 * g + r];
        auto step = [&](auto ic) {
            constexpr int i = kBack ? 15 - decltype(ic)::value : decltype(ic)::value;
            constexpr int gi = i % 4, ri = i / 4;
            double u[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) u[r] = un[r];
            if constexpr (kBack ? i > 0 : i + 1 < 16) {
#pragma unroll
                for (int r = 0; r < 4; ++r) un[r] = Ud[b][kBack ? i - 1 : i + 1][4 * g + r];
            }
            const double x = C[b][ri] * readlane_f64(rv, i);
            const double y = group_bcast<gi>(x);
            if (g == gi) C[b][ri] = x;
#pragma unroll
            for (int r = 0; r < 4; ++r) C[b][r] = __builtin_fma(-u[r], y, C[b][r]);
        };
        static_for<0, 16>(step);
#pragma unroll
        for (int b2 = 0; b2 < 8; ++b2) {
            if (kBack ? b2 >= b : b2 <= b) continue;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
                C[b2] = __builtin_amdgcn_mfma_f64_16x16x4f64(
                    Ut[kBack ? sub_tile(b2, b) : sub_tile(b, b2)][4 * kk + g][l & 15], C[b][kk],
                    C[b2], 0, 0, 0);
        }
    }
    if (!live) return;
#pragma unroll
    for (int b = 0; b < 8; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 16 * b + g + 4 * r;
            if (row < ib) X[at(row)] = C[b][r];
        }
}

// P <- U^-T P for the kb x kb upper factor U at Akk and the kb x T panel P (both column-major,
// leading dimension N), by recursive blocked substitution: the top h rows (h a multiple of 128,
// about half) are solved, their part of every lower row is subtracted with one FP64 MFMA product
// (K = h), and the bottom rows are solved; 128-row blocks are solved by k_panel_subst. The halving
// keeps most of the product work at large K, so each element of P is read and written about
// log2(kb / 128) times instead of once per 128-row block. Backward stable, unlike a solve through
// explicit inverses of the diagonal blocks, whose error grows with their condition number.
static int panel_solve(hipStream_t s, int64_t N, const double* Akk, int64_t kb, double* P,
                       int64_t T) {
    if (kb <= kPanelRows) {
        k_panel_subst<false, false><<<(unsigned)((T + 63) / 64), 256, 0, s>>>(N, Akk, (int)kb, P,
                                                                             T, N);
        GSDFT_HIP(hipGetLastError());
        return GSDFT_OK;
    }
    const int64_t h = (kb / kPanelRows + 1) / 2 * kPanelRows;
    GSDFT_TRY(panel_solve(s, N, Akk, h, P, T));
    // P(h + m, c) -= sum_{r < h} U(r, h + m) P(r, c)
    GSDFT_TRY(launch_gemm_tn_sub(kb - h, T, h, Akk + h * N, N, P, N, P + h, N, false, s));
    return panel_solve(s, N, Akk + h * N + h, kb - h, P + h, T);
}

namespace gsdft {

// K-slices for a coupling product of trsm_right_upper (output m x w, K = h): the deep levels of
// the halving have outputs of a few dozen 128 x 128 tiles (26 for RI-K's 3321 right-hand sides
// at K = 128), which leave most CUs idle. The count doubles until the tiles times the slices
// reach one workgroup per CU, each slice a multiple of 16 long and all of them within
// part_doubles.
static int64_t trsm_slices(int64_t m, int64_t w, int64_t h, int64_t part_doubles) {
    const int64_t tiles = ((m + 127) / 128) * ((w + 127) / 128);
    int64_t S = 1;
    while (S < 32 && S * tiles < 256 && (h / 16) % (2 * S) == 0 && h % 16 == 0 &&
           2 * S * m * w <= part_doubles)
        S *= 2;
    return S;
}

// X (m x n, column-major, leading dimension ldx) <- X U^-1, the solution of X U = B, or, with
// trans, X <- X U^-T, the solution of X U^T = B, for the n x n upper U (column-major, leading
// dimension ldu): the same recursive halving as panel_solve with the right-hand sides as X's rows
// (k_panel_subst with kRowRHS; kBack for U^T) and the coupling products on the general FP64 MFMA
// product, split over K (trsm_slices, summed in slice order) when `part` has room. Each row of X
// is solved by substitution in the order a row-by-row solve takes.
int trsm_right_upper(hipStream_t s, bool trans, int64_t n, const double* U, int64_t ldu,
                     double* X, int64_t m, int64_t ldx, double* part, int64_t part_doubles) {
    if (n <= 0 || m <= 0) return GSDFT_OK;
    if (n <= kPanelRows) {
        const unsigned blocks = (unsigned)((m + 63) / 64);
        if (trans)
            k_panel_subst<true, true><<<blocks, 256, 0, s>>>(ldu, U, (int)n, X, m, ldx);
        else
            k_panel_subst<false, true><<<blocks, 256, 0, s>>>(ldu, U, (int)n, X, m, ldx);
        GSDFT_HIP(hipGetLastError());
        return GSDFT_OK;
    }
    const int64_t h = (n / kPanelRows + 1) / 2 * kPanelRows;
    const double* U01 = U + h * ldu;                 // rows [0, h), columns [h, n)
    const double* U11 = U + h * ldu + h;
    if (!trans) {
        GSDFT_TRY(trsm_right_upper(s, false, h, U, ldu, X, m, ldx, part, part_doubles));
        // X(:, h:n) -= X(:, 0:h) U(0:h, h:n)
        GSDFT_TRY(gemm_cm_slices('N', 'N', m, n - h, h, -1.0, X, ldx, U01, ldu, 1.0, X + h * ldx,
                                 ldx, trsm_slices(m, n - h, h, part_doubles), part, s));
        return trsm_right_upper(s, false, n - h, U11, ldu, X + h * ldx, m, ldx, part,
                                part_doubles);
    }
    GSDFT_TRY(trsm_right_upper(s, true, n - h, U11, ldu, X + h * ldx, m, ldx, part,
                               part_doubles));
    // X(:, 0:h) -= X(:, h:n) U(0:h, h:n)^T
    GSDFT_TRY(gemm_cm_slices('N', 'T', m, h, n - h, -1.0, X + h * ldx, ldx, U01, ldu, 1.0, X, ldx,
                             trsm_slices(m, h, n - h, part_doubles), part, s));
    return trsm_right_upper(s, true, h, U, ldu, X, m, ldx, part, part_doubles);
}

}  // namespace gsdft

// C (T x T at C, leading dimension N) -= P^T P for the kb x T panel P, on the tiles on or above
// the diagonal (the sub-diagonal half of the diagonal tiles is formed too and never read).
static int trailing_update(hipStream_t s, int64_t N, const double* P, int64_t kb, double* C,
                           int64_t T) {
    return launch_gemm_tn_sub(T, T, kb, P, N, P, N, C, N, true, s);
}

// The diagonal block [k0, k0 + kb) of the column-major view: 128-row blocks factored by k_potf2,
// each block's panel solved and its trailing part of the block updated.
static int factor_diag_block(hipStream_t s, int64_t N, double* A, int64_t k0, int64_t kb,
                             int64_t* info) {
    double* Akk = A + k0 * N + k0;
    for (int64_t i0 = 0; i0 < kb; i0 += kPanelRows) {
        const int ib = (int)std::min((int64_t)kPanelRows, kb - i0);
        double* Aii = Akk + i0 * N + i0;
        k_potf2<<<1, kPotfThreads, 0, s>>>(N, Aii, ib, k0 + i0, info);
        GSDFT_HIP(hipGetLastError());
        const int64_t Ti = kb - i0 - ib;
        if (Ti == 0) break;
        double* Pi = Aii + (int64_t)ib * N;
        GSDFT_TRY(panel_solve(s, N, Aii, ib, Pi, Ti));
        GSDFT_TRY(trailing_update(s, N, Pi, ib, Pi + ib, Ti));
    }
    return GSDFT_OK;
}

// Right-looking blocked upper Cholesky of the column-major view A (= V, symmetric), A = U^T U, on
// two levels with the same three steps: for each diagonal block, factor it, solve the panel to its
// right (P = U_kk^-T A_k,rest) and update the trailing upper triangle (A_rest -= P^T P). The outer
// level uses kCholNb-row panels; each kCholNb diagonal block is factored the same way with 128-row
// blocks, whose factorisation is k_potf2. Every update is an FP64 MFMA product. *info receives the
// first failing leading minor (0 if none).
static int cholesky_blocked(hipStream_t s, int64_t N, double* A, int64_t* info) {
    k_info_reset<<<1, 1, 0, s>>>(info);
    GSDFT_HIP(hipGetLastError());
    for (int64_t k0 = 0; k0 < N; k0 += kCholNb) {
        const int64_t kb = std::min(kCholNb, N - k0);
        GSDFT_TRY(factor_diag_block(s, N, A, k0, kb, info));
        const int64_t T = N - k0 - kb;
        if (T == 0) break;
        double* P = A + (k0 + kb) * N + k0;
        GSDFT_TRY(panel_solve(s, N, A + k0 * N + k0, kb, P, T));
        GSDFT_TRY(trailing_update(s, N, P, kb, P + kb, T));
    }
    return GSDFT_OK;
}

extern "C" int gsdft_cholesky(int64_t N, double* V, void* workspace, size_t workspace_bytes,
                              void* stream) {
    if (N <= 0 || !V) return fail(GSDFT_ERR_ARG, "gsdft_cholesky: bad arguments");
    if ((N + 3) / 4 > 65535) return fail(GSDFT_ERR_ARG, "gsdft_cholesky: N too large");
    hipStream_t s = (hipStream_t)stream;
    Arena ar{(char*)workspace, workspace_bytes, 0};
    ar.take<double>(2 * N + 2);
    int64_t* info = ar.take<int64_t>(2);
    if (!info) return fail(GSDFT_ERR_WORKSPACE, "gsdft_cholesky: workspace too small");
    // Row-major lower L is column-major upper U = L^T, so factor the upper triangle (64-bit
    // offsets throughout: N * N exceeds the int32 range from N = 46341).
    {
        ProfileScope prof(kProfCholesky, s);
        GSDFT_TRY(cholesky_blocked(s, N, V, info));
    }
    dim3 grid((unsigned)((N + 63) / 64), (unsigned)((N + 3) / 4));
    k_zero_upper<<<grid, 256, 0, s>>>(N, V);
    GSDFT_HIP(hipGetLastError());
    int64_t h_info = 0;
    GSDFT_TRY(read_back(&h_info, info, sizeof(int64_t), s, "gsdft_cholesky: status"));
    if (h_info != 0)
        return fail(GSDFT_ERR_NOT_PD, "Cholesky: leading minor %lld of V + lam I is not positive "
                    "definite", (long long)h_info);
    return GSDFT_OK;
}

// Zeroes the strict upper triangle (row-major) of the 128 x 128 diagonal tiles: the only
// entries above the diagonal that the factorisation writes (the sub-diagonal half of its
// column-major diagonal tiles, formed by the updates and never read), when the metric was formed
// with zeros above the diagonal.
__global__ void k_zero_diag_tiles(int64_t N, double* __restrict__ V) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    const int64_t p = t / kPanelRows;
    if (p >= N) return;
    const int64_t q = (p / kPanelRows) * kPanelRows + t % kPanelRows;
    if (q > p && q < N) V[p * N + q] = 0.0;
}

extern "C" int gsdft_aux_cholesky(int64_t N, const double* log_alpha, const double* aux_centers,
                                  double lam, double omega, double* L, void* workspace,
                                  size_t workspace_bytes, void* stream) {
    if (N <= 0 || !log_alpha || !aux_centers || !L)
        return fail(GSDFT_ERR_ARG, "gsdft_aux_cholesky: bad arguments");
    if (!(omega >= 0.0) || std::isinf(omega))
        return fail(GSDFT_ERR_ARG, "gsdft_aux_cholesky: omega must be finite and >= 0");
    if ((N + 3) / 4 > 65535) return fail(GSDFT_ERR_ARG, "gsdft_aux_cholesky: N too large");
    hipStream_t s = (hipStream_t)stream;
    Arena ar{(char*)workspace, workspace_bytes, 0};
    double* bk = ar.take<double>(2 * N + 2);
    int64_t* info = ar.take<int64_t>(2);
    if (!info) return fail(GSDFT_ERR_WORKSPACE, "gsdft_aux_cholesky: workspace too small");
    k_aux_prep<<<blocks_for(N, 256), 256, 0, s>>>(N, log_alpha, bk, bk + N);
    dim3 grid((unsigned)((N + 63) / 64), (unsigned)((N + 4 * kMetricRows - 1) / (4 * kMetricRows)));
    profile_begin(kProfMetric, s);
    k_metric<true><<<grid, 256, 0, s>>>(N, bk, bk + N, aux_centers, lam, omega, L);
    profile_end(kProfMetric, s);
    GSDFT_HIP(hipGetLastError());
    {
        ProfileScope prof(kProfCholesky, s);
        GSDFT_TRY(cholesky_blocked(s, N, L, info));
    }
    k_zero_diag_tiles<<<blocks_for(N * kPanelRows, 256), 256, 0, s>>>(N, L);
    GSDFT_HIP(hipGetLastError());
    int64_t h_info = 0;
    GSDFT_TRY(read_back(&h_info, info, sizeof(int64_t), s, "gsdft_aux_cholesky: status"));
    if (h_info != 0)
        return fail(GSDFT_ERR_NOT_PD, "Cholesky: leading minor %lld of V + lam I is not positive "
                    "definite", (long long)h_info);
    return GSDFT_OK;
}

extern "C" int gsdft_cho_solve(int64_t N, const double* L, const double* gamma, double* d,
                               double* energy, void* stream) {
    if (N <= 0 || !L || !gamma || !d) return fail(GSDFT_ERR_ARG, "gsdft_cho_solve: bad arguments");
    hipStream_t s = (hipStream_t)stream;
    GSDFT_HIP(hipMemcpyAsync(d, gamma, sizeof(double) * N, hipMemcpyDeviceToDevice, s));
    {
        ProfileScope prof(kProfSolve, s);
        GSDFT_TRY(launch_trsv_pair(N, L, d, s));
    }
    if (energy) {
        k_scaled_dot<<<1, 1024, 0, s>>>(N, gamma, d, 0.5, energy);
        GSDFT_HIP(hipGetLastError());
    }
    return GSDFT_OK;
}

extern "C" int gsdft_gamma_workspace_size(int64_t M, int64_t k, int64_t N, int64_t n,
                                          size_t* bytes) {
    (void)k;
    if (M < 0 || N < 0 || n < 0 || !bytes) return fail(GSDFT_ERR_ARG, "gamma_workspace_size: bad arguments");
    GSDFT_TRY(check_pairs(n, "gamma_workspace_size"));
    Arena ar{nullptr, 0, 0};
    GammaWs w;
    GSDFT_TRY(layout_gamma(ar, M, N, n, false, &w));
    *bytes = ar.need();
    return GSDFT_OK;
}

extern "C" int gsdft_gamma_vjp_workspace_size(int64_t M, int64_t k, int64_t N, int64_t n,
                                              size_t* bytes) {
    (void)k;
    if (M < 0 || N < 0 || n < 0 || !bytes) return fail(GSDFT_ERR_ARG, "gamma_vjp_workspace_size: bad arguments");
    GSDFT_TRY(check_pairs(n, "gamma_vjp_workspace_size"));
    Arena ar{nullptr, 0, 0};
    GammaWs w;
    GSDFT_TRY(layout_gamma(ar, M, N, n, true, &w));
    *bytes = ar.need();
    return GSDFT_OK;
}

namespace {

// gsdft_gamma's body over a workspace of `bytes` bytes; `profile` records the kernel timer
// (HIP events, created on demand) and the node counter.
int gamma_run(int64_t M, const double* quat, const double* log_scale, const double* centers,
              int64_t k, const double* C, const double* occ, int64_t N, const double* log_alpha,
              const double* aux_centers, int64_t n, const int32_t* pi, const int32_t* pj,
              const double* weight, double* gamma, void* workspace, size_t bytes, hipStream_t s,
              bool profile) {
    Arena ar{(char*)workspace, bytes, 0};
    GammaWs w;
    GSDFT_TRY(layout_gamma(ar, M, N, n, false, &w));
    if (!w.partial) return fail(GSDFT_ERR_WORKSPACE, "gsdft_gamma: workspace too small");
    if (n == 0) {
        k_fill<<<blocks_for(N, 256), 256, 0, s>>>(N, 0.0, gamma);
        GSDFT_HIP(hipGetLastError());
        return GSDFT_OK;
    }
    GSDFT_TRY(gamma_prologue(M, quat, log_scale, centers, k, C, occ, N, log_alpha, n, pi, pj,
                             weight, w, s));
    const int64_t G = (N % M == 0) ? N / M : 1;          // scales per centre of a product aux
    k_aux_bwd_prep<<<blocks_for(N, 256), 256, 0, s>>>(N, G, w.beta, w.kn, aux_centers, nullptr,
                                                      nullptr, kAuxForward, coulomb_table(),
                                                      w.aux);
    GSDFT_HIP(hipGetLastError());
    GSDFT_TRY(launch_pair_order(n, w.rec, kRec, w.pair_order, s));
    k_rec_gather<<<blocks_for(n * kRec, 256), 256, 0, s>>>(n, w.pair_order.perm, w.rec,
                                                            w.rec_sorted);
    GSDFT_HIP(hipGetLastError());
    const int64_t groups = (n + kFwdPairs - 1) / kFwdPairs;
    const int64_t nrb = (N + kFwdRecs - 1) / kFwdRecs;
    if (nrb * 256 > (int64_t)UINT32_MAX || groups > kMaxGridY)
        return fail(GSDFT_ERR_ARG, "gsdft_gamma: N_aux = %lld or n = %lld too large for one launch",
                    (long long)N, (long long)n);
    const dim3 grid((unsigned)nrb, (unsigned)groups);
    if (profile) profile_begin(kProfGammaFwd, s);
    k_gamma_fwd_pairs<<<grid, 256, 0, s>>>(n, w.rec_sorted, N, w.aux, w.partial,
                                           profile ? profile_work_counter(kProfGammaFwd)
                                                   : nullptr);
    if (profile) profile_end(kProfGammaFwd, s);
    GSDFT_HIP(hipGetLastError());
    k_slot_sum<<<blocks_for(N, 256), 256, 0, s>>>(N, G, groups, w.partial, gamma);
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}

// Static scratch of gsdft_gamma_noalloc: one copy per device, held while the process runs. Host
// code never names it in a launch or copy: its device address comes from hipGetSymbolAddress, once
// per device, with that device current.
constexpr size_t kScratchBytes = size_t(64) << 20;
__device__ __align__(256) char scratch[kScratchBytes];

std::mutex g_scratch_mu;
std::vector<void*> g_scratch_ptr;      // device address of `scratch`, by device id

int scratch_address(void** out) {
    int dev = 0;
    GSDFT_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if ((int)g_scratch_ptr.size() <= dev) g_scratch_ptr.resize(dev + 1, nullptr);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (!p) return fail(GSDFT_ERR_HIP, "hipGetSymbolAddress(scratch) gave a null address");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return GSDFT_OK;
}

}  // namespace

extern "C" int gsdft_gamma(int64_t M, const double* quat, const double* log_scale,
                           const double* centers, int64_t k, const double* C, const double* occ,
                           int64_t N, const double* log_alpha, const double* aux_centers,
                           int64_t n, const int32_t* pi, const int32_t* pj, const double* weight,
                           double* gamma, void* workspace, size_t workspace_bytes, void* stream) {
    if (M <= 0 || N <= 0 || n < 0 || k <= 0 || !gamma)
        return fail(GSDFT_ERR_ARG, "gsdft_gamma: bad arguments");
    GSDFT_TRY(check_pairs(n, "gsdft_gamma"));
    return gamma_run(M, quat, log_scale, centers, k, C, occ, N, log_alpha, aux_centers, n, pi, pj,
                     weight, gamma, workspace, workspace_bytes, (hipStream_t)stream, true);
}

extern "C" int gsdft_gamma_noalloc(int64_t M, const double* quat, const double* log_scale,
                                   const double* centers, int64_t k, const double* C,
                                   const double* occ, int64_t N, const double* log_alpha,
                                   const double* aux_centers, int64_t n, const int32_t* pi,
                                   const int32_t* pj, const double* weight, double* gamma,
                                   void* stream) {
    if (M <= 0 || N <= 0 || n < 0 || k <= 0 || !gamma)
        return fail(GSDFT_ERR_ARG, "gsdft_gamma_noalloc: bad arguments");
    GSDFT_TRY(check_pairs(n, "gsdft_gamma_noalloc"));
    Arena ar{nullptr, 0, 0};
    GammaWs w;
    GSDFT_TRY(layout_gamma(ar, M, N, n, false, &w));
    if (ar.need() > kScratchBytes)
        return fail(GSDFT_ERR_ARG, "gsdft_gamma_noalloc: M = %lld, N_aux = %lld, n = %lld need "
                    "%zu bytes of scratch; the static scratch holds %zu (use gsdft_gamma with a "
                    "workspace)", (long long)M, (long long)N, (long long)n, ar.need(),
                    kScratchBytes);
    void* p = nullptr;
    GSDFT_TRY(scratch_address(&p));
    return gamma_run(M, quat, log_scale, centers, k, C, occ, N, log_alpha, aux_centers, n, pi, pj,
                     weight, gamma, p, kScratchBytes, (hipStream_t)stream, false);
}

extern "C" int gsdft_gamma_vjp(int64_t M, const double* quat, const double* log_scale,
                               const double* centers, int64_t k, const double* C,
                               const double* occ, int64_t N, const double* log_alpha,
                               const double* aux_centers, int64_t n, const int32_t* pi,
                               const int32_t* pj, const double* weight, const int32_t* row_ptr,
                               const int32_t* row_perm, const int32_t* col_ptr,
                               const int32_t* col_perm, const double* dgamma,
                               const double* dgamma_scale, double* J, double* dquat,
                               double* dlog_scale, double* dcenters, double* dC, void* workspace,
                               size_t workspace_bytes, void* stream) {
    if (M <= 0 || N <= 0 || n < 0 || k <= 0 || !dgamma || !dquat || !dlog_scale || !dcenters ||
        !dC || !row_ptr || !col_ptr || (n > 0 && (!J || !row_perm || !col_perm)))
        return fail(GSDFT_ERR_ARG, "gsdft_gamma_vjp: bad arguments");
    GSDFT_TRY(check_pairs(n, "gsdft_gamma_vjp"));
    hipStream_t s = (hipStream_t)stream;
    Arena ar{(char*)workspace, workspace_bytes, 0};
    GammaWs w;
    GSDFT_TRY(layout_gamma(ar, M, N, n, true, &w));
    if (!w.contrib) return fail(GSDFT_ERR_WORKSPACE, "gsdft_gamma_vjp: workspace too small");
    GSDFT_TRY(gamma_prologue(M, quat, log_scale, centers, k, C, occ, N, log_alpha, n, pi, pj,
                             weight, w, s));
    if (n > 0) {
        const int64_t G = (N % M == 0) ? N / M : 1;      // scales per centre of a product aux
        k_aux_bwd_prep<<<blocks_for(N, 256), 256, 0, s>>>(N, G, w.beta, w.kn, aux_centers,
                                                          dgamma, dgamma_scale, kAuxFoldU,
                                                          coulomb_table(),
                                                          w.aux);
        GSDFT_TRY(launch_pair_order(n, w.rec, kRec, w.pair_order, s));
        k_rec_gather<<<blocks_for(n * kRec, 256), 256, 0, s>>>(n, w.pair_order.perm, w.rec,
                                                                w.rec_sorted);
        const Split sp = bwd_split_records(N, n);
        const int64_t per_launch = bwd_slabs_per_launch(N, n);
        profile_begin(kProfGammaBwd, s);
        for (int64_t sl = 0; sl < sp.slabs; sl += per_launch) {
            const int64_t r = std::min(per_launch, sp.slabs - sl);
            dim3 grid((unsigned)((n + 255) / 256), (unsigned)r);
            k_gamma_bwd<false, false, true><<<grid, 256, 0, s>>>(
                n, w.rec_sorted, N, w.aux, sp.per_slab, w.acc,
                profile_work_counter(kProfGammaBwd), nullptr, 0, nullptr, nullptr, nullptr,
                nullptr, 0, sl, sl == 0 ? 1 : 0);
            GSDFT_HIP(hipGetLastError());
            if (r > 1) {
                k_slab_fold<<<blocks_for(n * kAcc, 256), 256, 0, s>>>(n, r, w.acc);
                GSDFT_HIP(hipGetLastError());
            }
        }
        profile_end(kProfGammaBwd, s);
        k_pair_finalize<<<blocks_for(n, 256), 256, 0, s>>>(n, n, 1, kPref3c,
                                                           w.pair_order.perm, pi, pj, weight,
                                                           w.A6, centers, w.Nrm, w.rec_sorted,
                                                           w.acc, J, w.contrib);
        GSDFT_HIP(hipGetLastError());
    }
    k_splat_grad<<<blocks_for(M * 64, 256), 256, 0, s>>>(M, n, row_ptr, row_perm, col_ptr,
                                                         col_perm, w.contrib, quat, log_scale,
                                                         dquat, dlog_scale, dcenters);
    GSDFT_TRY(launch_dC(M, k, row_ptr, row_perm, col_ptr, col_perm, pi, pj, J, weight, C, occ, dC,
                        s));
    return GSDFT_OK;
}

// ------------------------------------------------------------------ nuclear attraction (C ABI)

namespace gsdft {
namespace {

struct ExternalWs {
    GammaWs g;
    double* atom_partial;       // (pair blocks, n_atoms, 3) from the pair pass
    double* atom_groups;        // (ceil(pair blocks / 256), n_atoms, 3)
    double* dot_part;           // dot_blocks(n)
};

constexpr int64_t kAtomGroup = 256;   // pair blocks per first-stage sum of the nuclear forces

inline int64_t pair_blocks(int64_t n) { return n > 0 ? (n + 255) / 256 : 1; }

int layout_external(Arena& ar, int64_t M, int64_t n, int64_t n_atoms, ExternalWs* w) {
    GSDFT_TRY(layout_gamma(ar, M, n_atoms, n, true, &w->g));
    const int64_t blocks = pair_blocks(n);
    w->atom_partial = ar.take<double>(blocks * n_atoms * 3 + 3);
    w->atom_groups = ar.take<double>(((blocks + kAtomGroup - 1) / kAtomGroup) * n_atoms * 3 + 3);
    w->dot_part = ar.take<double>(dot_blocks(n));
    return GSDFT_OK;
}

// out[g][i] = sum of part[b][i] over the pair blocks b of group g (kAtomGroup each), in order.
__global__ void k_atom_sum_groups(int64_t count, int64_t blocks, const double* __restrict__ part,
                                  double* __restrict__ out) {
    const int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    const int64_t groups = (blocks + kAtomGroup - 1) / kAtomGroup;
    if (t >= groups * count) return;
    const int64_t g = t / count, i = t % count;
    const int64_t b1 = min(blocks, (g + 1) * kAtomGroup);
    double s = 0.0;
    for (int64_t b = g * kAtomGroup; b < b1; ++b) s += part[b * count + i];
    out[g * count + i] = s;
}

// datoms[A][c] = -Z_A 2 pi sum_g groups[g][A][c], in group order.
__global__ void k_atom_force_finish(int64_t n_atoms, int64_t groups,
                                    const double* __restrict__ gsum,
                                    const double* __restrict__ charges,
                                    double* __restrict__ datoms) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= 3 * n_atoms) return;
    double s = 0.0;
    for (int64_t g = 0; g < groups; ++g) s += gsum[g * 3 * n_atoms + i];
    datoms[i] = -charges[i / 3] * kPrefNuc * s;
}

// V (n) = the nuclear attraction of every listed pair (J of the reverse kernel with the nuclei as
// point-charge records) and, for a non-null C, the slot moments behind its gradient.
int external_pass(int64_t M, const double* quat, const double* log_scale, const double* centers,
                  int64_t k, const double* C, const double* occ, int64_t n, const int32_t* pi,
                  const int32_t* pj, const double* weight, int64_t n_atoms,
                  const double* atom_coords, const double* atom_charges, double* V,
                  ExternalWs& w, bool atom_forces, hipStream_t s) {
    GSDFT_TRY(gamma_prologue(M, quat, log_scale, centers, k, C, occ, n_atoms, nullptr, n, pi, pj,
                             weight, w.g, s));
    k_atom_rec<<<blocks_for(n_atoms, 256), 256, 0, s>>>(n_atoms, atom_coords, atom_charges,
                                                        w.g.aux);
    GSDFT_HIP(hipGetLastError());
    GSDFT_TRY(launch_pair_order(n, w.g.rec, kRec, w.g.pair_order, s));
    k_rec_gather<<<blocks_for(n * kRec, 256), 256, 0, s>>>(n, w.g.pair_order.perm, w.g.rec,
                                                            w.g.rec_sorted);
    const Split sp = bwd_split(n_atoms, n);
    dim3 grid((unsigned)((n + 255) / 256), (unsigned)sp.slabs);
    profile_begin(kProfNucPairs, s);
    if (atom_forces)
        k_gamma_bwd<false, true><<<grid, 256, 0, s>>>(n, w.g.rec_sorted, n_atoms, w.g.aux,
                                                      sp.per_slab, w.g.acc,
                                                      profile_work_counter(kProfNucPairs),
                                                      nullptr, 0, w.atom_partial, nullptr, nullptr, nullptr);
    else
        k_gamma_bwd<false><<<grid, 256, 0, s>>>(n, w.g.rec_sorted, n_atoms, w.g.aux, sp.per_slab,
                                                w.g.acc, profile_work_counter(kProfNucPairs),
                                                nullptr, 0, nullptr, nullptr, nullptr, nullptr);
    profile_end(kProfNucPairs, s);
    GSDFT_HIP(hipGetLastError());
    k_pair_finalize<<<blocks_for(n, 256), 256, 0, s>>>(n, n, sp.slabs, kPrefNuc,
                                                       w.g.pair_order.perm, pi, pj, weight,
                                                       w.g.A6, centers, w.g.Nrm, w.g.rec_sorted,
                                                       w.g.acc, V, w.g.contrib);
    GSDFT_HIP(hipGetLastError());
    return GSDFT_OK;
}

int check_atoms(int64_t n_atoms, const double* coords, const double* charges) {
    if (n_atoms <= 0 || !coords || !charges)
        return fail(GSDFT_ERR_ARG, "nuclear attraction: need n_atoms > 0, coordinates and charges");
    return GSDFT_OK;
}

}  // namespace
}  // namespace gsdft

extern "C" int gsdft_external_workspace_size(int64_t M, int64_t k, int64_t n, int64_t n_atoms,
                                             size_t* bytes) {
    (void)k;
    if (M < 0 || n < 0 || n_atoms < 0 || !bytes)
        return fail(GSDFT_ERR_ARG, "external_workspace_size: bad arguments");
    GSDFT_TRY(check_pairs(n, "external_workspace_size"));
    Arena ar{nullptr, 0, 0};
    ExternalWs w;
    GSDFT_TRY(layout_external(ar, M, n, n_atoms, &w));
    *bytes = ar.need();
    return GSDFT_OK;
}

extern "C" int gsdft_nuclear_pairs(int64_t M, const double* quat, const double* log_scale,
                                   const double* centers, int64_t n, const int32_t* pi,
                                   const int32_t* pj, int64_t n_atoms, const double* atom_coords,
                                   const double* atom_charges, double* V, void* workspace,
                                   size_t workspace_bytes, void* stream) {
    if (M <= 0 || n < 0 || (n > 0 && (!pi || !pj || !V)))
        return fail(GSDFT_ERR_ARG, "gsdft_nuclear_pairs: bad arguments");
    GSDFT_TRY(check_pairs(n, "gsdft_nuclear_pairs"));
    GSDFT_TRY(check_atoms(n_atoms, atom_coords, atom_charges));
    if (n == 0) return GSDFT_OK;
    hipStream_t s = (hipStream_t)stream;
    Arena ar{(char*)workspace, workspace_bytes, 0};
    ExternalWs w;
    GSDFT_TRY(layout_external(ar, M, n, n_atoms, &w));
    if (!w.atom_partial) return fail(GSDFT_ERR_WORKSPACE, "gsdft_nuclear_pairs: workspace too small");
    return external_pass(M, quat, log_scale, centers, 0, nullptr, nullptr, n, pi, pj, nullptr,
                         n_atoms, atom_coords, atom_charges, V, w, false, s);
}

extern "C" int gsdft_external_energy(
    int64_t M, const double* quat, const double* log_scale, const double* centers, int64_t k,
    const double* C, const double* occ, int64_t n, const int32_t* pi, const int32_t* pj,
    const double* weight, const int32_t* row_ptr, const int32_t* row_perm,
    const int32_t* col_ptr, const int32_t* col_perm, int64_t n_atoms, const double* atom_coords,
    const double* atom_charges, double* energy, double* V, double* dquat, double* dlog_scale,
    double* dcenters, double* dC, double* datoms, void* workspace, size_t workspace_bytes,
    void* stream) {
    const bool splat_grad = dquat || dlog_scale || dcenters || dC;
    if (M <= 0 || n < 0 || k <= 0 || !C || !occ || !energy || (n > 0 && (!pi || !pj || !weight || !V)))
        return fail(GSDFT_ERR_ARG, "gsdft_external_energy: bad arguments");
    GSDFT_TRY(check_pairs(n, "gsdft_external_energy"));
    if (splat_grad && (!dquat || !dlog_scale || !dcenters || !dC || !row_ptr || !col_ptr ||
                       (n > 0 && (!row_perm || !col_perm))))
        return fail(GSDFT_ERR_ARG, "gsdft_external_energy: the splat gradients come together "
                    "(dquat, dlog_scale, dcenters, dC) and need the pair index");
    GSDFT_TRY(check_atoms(n_atoms, atom_coords, atom_charges));
    hipStream_t s = (hipStream_t)stream;
    Arena ar{(char*)workspace, workspace_bytes, 0};
    ExternalWs w;
    GSDFT_TRY(layout_external(ar, M, n, n_atoms, &w));
    if (!w.atom_partial) return fail(GSDFT_ERR_WORKSPACE, "gsdft_external_energy: workspace too small");
    if (n == 0) {
        k_fill<<<1, 256, 0, s>>>(1, 0.0, energy);
        if (splat_grad) {
            k_fill<<<blocks_for(4 * M, 256), 256, 0, s>>>(4 * M, 0.0, dquat);
            k_fill<<<blocks_for(3 * M, 256), 256, 0, s>>>(3 * M, 0.0, dlog_scale);
            k_fill<<<blocks_for(3 * M, 256), 256, 0, s>>>(3 * M, 0.0, dcenters);
            k_fill<<<blocks_for(M * k, 256), 256, 0, s>>>(M * k, 0.0, dC);
        }
        if (datoms) k_fill<<<blocks_for(3 * n_atoms, 256), 256, 0, s>>>(3 * n_atoms, 0.0, datoms);
        GSDFT_HIP(hipGetLastError());
        return GSDFT_OK;
    }
    GSDFT_TRY(external_pass(M, quat, log_scale, centers, k, C, occ, n, pi, pj, weight, n_atoms,
                            atom_coords, atom_charges, V, w, datoms != nullptr, s));
    // E = sum_a q_a V_a (gs_dft/screening/pairs.py:429-432), fixed summation order
    GSDFT_TRY(launch_scaled_dot(n, w.g.q, V, 1.0, energy, w.dot_part, s));
    if (splat_grad) {
        k_splat_grad<<<blocks_for(M * 64, 256), 256, 0, s>>>(M, n, row_ptr, row_perm, col_ptr,
                                                             col_perm, w.g.contrib, quat,
                                                             log_scale, dquat, dlog_scale,
                                                             dcenters);
        GSDFT_HIP(hipGetLastError());
        GSDFT_TRY(launch_dC(M, k, row_ptr, row_perm, col_ptr, col_perm, pi, pj, V, weight, C, occ,
                            dC, s));
    }
    if (datoms) {
        // the pair pass left each pair block's force on every nucleus: sum them in fixed order
        const int64_t blocks = pair_blocks(n), groups = (blocks + kAtomGroup - 1) / kAtomGroup;
        profile_begin(kProfNucAtoms, s);
        k_atom_sum_groups<<<blocks_for(groups * 3 * n_atoms, 256), 256, 0, s>>>(
            3 * n_atoms, blocks, w.atom_partial, w.atom_groups);
        k_atom_force_finish<<<blocks_for(3 * n_atoms, 256), 256, 0, s>>>(
            n_atoms, groups, w.atom_groups, atom_charges, datoms);
        profile_end(kProfNucAtoms, s);
        GSDFT_HIP(hipGetLastError());
    }
    return GSDFT_OK;
}

extern "C" int gsdft_density_pairs(int64_t n, const int32_t* pi, const int32_t* pj, int64_t k,
                                   const double* C, const double* occ, double* out,
                                   void* stream) {
    if (n < 0 || k <= 0 || (n > 0 && (!pi || !pj || !C || !occ || !out)))
        return fail(GSDFT_ERR_ARG, "gsdft_density_pairs: bad arguments");
    GSDFT_TRY(check_pairs(n, "gsdft_density_pairs"));
    return launch_pair_density(n, pi, pj, nullptr, k, C, occ, out, (hipStream_t)stream);
}

// ------------------------------------------------------------------ exact Coulomb (C ABI)

namespace gsdft {
namespace {

struct EriWs {
    double *A6, *Nrm, *q, *rec3, *rec, *partial, *contrib;
    double *jacc, *bra_part, *ket_part;     // symmetric passes (jacc: J, or the ten moments)
    double* dot_part;                       // dot_blocks(n)
    int64_t band;
    PairOrderWs order;
};

// Bra band height of the symmetric forward: a multiple of 256, at most 16384, with the band's
// ket partials ((band / 256) x n doubles) within 1 GiB.
int64_t eri_band(int64_t n) {
    const int64_t groups_cap = std::max<int64_t>(1, ((int64_t)1 << 27) / std::max<int64_t>(n, 1));
    int64_t groups = std::min<int64_t>({(n + 255) / 256, 64, groups_cap});
    return std::max<int64_t>(groups, 1) * 256;
}

// The same for the reverse, whose ket partials are (band / 64) x 10 x n doubles, within 8 GiB
// (fewer, fuller band launches: the reverse is the longer pass).
int64_t eri_band10(int64_t n) {
    const int64_t waves_cap = ((int64_t)1 << 30) / (kEriAcc * std::max<int64_t>(n, 1));
    const int64_t groups = std::min<int64_t>({(n + 255) / 256, 64, waves_cap / 4});
    return std::max<int64_t>(groups, 1) * 256;
}

int layout_eri(Arena& ar, int64_t M, int64_t n, bool grads, EriWs* w) {
    w->A6 = ar.take<double>(6 * M + 1);
    w->Nrm = ar.take<double>(M + 1);
    w->q = ar.take<double>(n + 1);
    w->rec3 = ar.take<double>(kRec * n + kRec);
    w->rec = ar.take<double>(kEriRec * n + kEriRec);
    GSDFT_TRY(pair_order_layout(ar, n, &w->order));
    w->dot_part = ar.take<double>(dot_blocks(n));
    w->jacc = w->bra_part = w->ket_part = nullptr;
    w->band = 0;
    if (grads) {
        w->band = eri_band10(n);
        const int64_t slabs = (n + kEriSymSlabB - 1) / kEriSymSlabB;
        w->jacc = ar.take<double>(kEriAcc * n + 1);
        w->bra_part = ar.take<double>(slabs * kEriAcc * w->band + 1);
        w->ket_part = ar.take<double>((w->band / 64) * kEriAcc * n + 1);
        w->partial = w->jacc;
        w->contrib = ar.take<double>(20 * n + 1);
    } else {
        w->band = eri_band(n);
        const int64_t slabs = (n + kEriSymSlab - 1) / kEriSymSlab;
        w->jacc = ar.take<double>(n + 1);
        w->bra_part = ar.take<double>(slabs * w->band + 1);
        w->ket_part = ar.take<double>((w->band / 256) * n + 1);
        w->partial = w->jacc;
        w->contrib = nullptr;
    }
    return GSDFT_OK;
}

}  // namespace
}  // namespace gsdft

extern "C" int gsdft_exact_coulomb_workspace_size(int64_t M, int64_t k, int64_t n, int grads,
                                                  size_t* bytes) {
    (void)k;
    if (M < 0 || n < 0 || !bytes)
        return fail(GSDFT_ERR_ARG, "exact_coulomb_workspace_size: bad arguments");
    GSDFT_TRY(check_pairs(n, "exact_coulomb_workspace_size"));
    Arena ar{nullptr, 0, 0};
    EriWs w;
    GSDFT_TRY(layout_eri(ar, M, n, grads != 0, &w));
    *bytes = ar.need();
    return GSDFT_OK;
}

namespace gsdft {
namespace {

// Pw_a = w_a P[i_a][j_a] for a row-major (M, M) density matrix P.
__global__ void k_pair_gather_density(int64_t n, int64_t M, const int32_t* __restrict__ pi,
                                      const int32_t* __restrict__ pj,
                                      const double* __restrict__ weight,
                                      const double* __restrict__ P, double* __restrict__ q) {
    const int64_t a = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (a >= n) return;
    q[a] = weight[a] * P[(int64_t)pi[a] * M + pj[a]];
}

// dP (M, M, zeroed beforehand) = the Coulomb matrix on the listed entries: dP[i_a][j_a] = J_a
// and, with sym, dP[j_a][i_a] = J_a too (gs_dft/coulomb/stream.py:127-134); dead entries are
// skipped. The live entries name distinct pairs, so no two threads write one element.
__global__ void k_scatter_density_grad(int64_t n, int64_t M, const int32_t* __restrict__ pi,
                                       const int32_t* __restrict__ pj,
                                       const double* __restrict__ weight,
                                       const double* __restrict__ J, int sym,
                                       double* __restrict__ dP) {
    const int64_t a = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (a >= n || weight[a] == 0.0) return;
    const int64_t i = pi[a], j = pj[a];
    dP[i * M + j] = J[a];
    if (sym && i != j) dP[j * M + i] = J[a];
}

// The density source of the exact Coulomb: occupied orbitals (Pw_a = w_a sum_o occ_o C_io C_jo,
// gradient dC) or a density matrix (Pw_a = w_a P_ij, gradient dP).
struct ExactDensity {
    int64_t k;
    const double *C, *occ, *P;
    int sym;
    double *dC, *dP;
};

int exact_run(int64_t M, const double* quat, const double* log_scale, const double* centers,
              const ExactDensity& den, int64_t n, const int32_t* pi, const int32_t* pj,
              const double* weight, const int32_t* row_ptr, const int32_t* row_perm,
              const int32_t* col_ptr, const int32_t* col_perm, double* energy, double* J,
              double* dquat, double* dlog_scale, double* dcenters, bool grads, void* workspace,
              size_t workspace_bytes, hipStream_t s, const char* name) {
    if (n > INT32_MAX) return fail(GSDFT_ERR_ARG, "%s: n exceeds the int32 range", name);
    Arena ar{(char*)workspace, workspace_bytes, 0};
    EriWs w;
    GSDFT_TRY(layout_eri(ar, M, n, grads, &w));
    if (!w.partial || (grads && !w.contrib))
        return fail(GSDFT_ERR_WORKSPACE, "%s: workspace too small", name);
    if (den.dP) {
        k_fill<<<blocks_for(M * M, 256), 256, 0, s>>>(M * M, 0.0, den.dP);
        GSDFT_HIP(hipGetLastError());
    }
    if (n == 0) {
        k_fill<<<1, 256, 0, s>>>(1, 0.0, energy);
        if (grads) {
            k_fill<<<blocks_for(4 * M, 256), 256, 0, s>>>(4 * M, 0.0, dquat);
            k_fill<<<blocks_for(3 * M, 256), 256, 0, s>>>(3 * M, 0.0, dlog_scale);
            k_fill<<<blocks_for(3 * M, 256), 256, 0, s>>>(3 * M, 0.0, dcenters);
            if (den.dC)
                k_fill<<<blocks_for(M * den.k, 256), 256, 0, s>>>(M * den.k, 0.0, den.dC);
        }
        GSDFT_HIP(hipGetLastError());
        return GSDFT_OK;
    }
    GSDFT_TRY(launch_chart(M, quat, log_scale, w.A6, w.Nrm, s));
    if (den.P) {
        k_pair_gather_density<<<blocks_for(n, 256), 256, 0, s>>>(n, M, pi, pj, weight, den.P,
                                                                 w.q);
        GSDFT_HIP(hipGetLastError());
    } else {
        GSDFT_TRY(launch_pair_density(n, pi, pj, weight, den.k, den.C, den.occ, w.q, s));
    }
    k_pair_rec<<<blocks_for(n, 256), 256, 0, s>>>(n, pi, pj, w.A6, centers, w.Nrm, w.q, w.rec3);
    GSDFT_HIP(hipGetLastError());
    GSDFT_TRY(launch_pair_order(n, w.rec3, kRec, w.order, s));
    k_eri_rec<<<blocks_for(n, 256), 256, 0, s>>>(n, w.order.perm, pi, pj, w.A6, centers, w.Nrm,
                                                 w.q, weight, w.rec);
    GSDFT_HIP(hipGetLastError());
    if (!grads) {
        // bands of bra slots, each against the kets from its own start on
        if ((n + kEriSymSlab - 1) / kEriSymSlab > 65535)
            return fail(GSDFT_ERR_ARG, "%s: n exceeds the supported %lld pairs", name,
                        (long long)65535 * kEriSymSlab);
        k_fill<<<blocks_for(n, 256), 256, 0, s>>>(n, 0.0, w.jacc);
        profile_begin(kProfEriFwd, s);
        for (int64_t A0 = 0; A0 < n; A0 += w.band) {
            const int64_t hb = std::min(w.band, n - A0);
            dim3 g((unsigned)((hb + 255) / 256),
                   (unsigned)((n - A0 + kEriSymSlab - 1) / kEriSymSlab));
            k_eri_fwd_sym<<<g, 256, 0, s>>>(n, w.rec, A0, w.band, w.bra_part, w.ket_part,
                                            profile_work_counter(kProfEriFwd));
            k_eri_sym_reduce<<<blocks_for(n - A0, 256), 256, 0, s>>>(
                n, A0, w.band, g.x, g.y, w.band, w.bra_part, w.ket_part, w.jacc);
        }
        profile_end(kProfEriFwd, s);
        GSDFT_HIP(hipGetLastError());
        k_eri_finish<<<blocks_for(n, 256), 256, 0, s>>>(n, 1, w.order.perm, w.rec, w.jacc, J);
    } else {
        if ((n + kEriSymSlabB - 1) / kEriSymSlabB > 65535)
            return fail(GSDFT_ERR_ARG, "%s: n exceeds the supported %lld pairs", name,
                        (long long)65535 * kEriSymSlabB);
        k_fill<<<blocks_for(kEriAcc * n, 256), 256, 0, s>>>(kEriAcc * n, 0.0, w.jacc);
        profile_begin(kProfEriBwd, s);
        for (int64_t A0 = 0; A0 < n; A0 += w.band) {
            const int64_t hb = std::min(w.band, n - A0);
            dim3 g((unsigned)((hb + 255) / 256),
                   (unsigned)((n - A0 + kEriSymSlabB - 1) / kEriSymSlabB));
            k_eri_bwd_sym<<<g, 256, 0, s>>>(n, w.rec, A0, w.band, w.bra_part, w.ket_part,
                                            profile_work_counter(kProfEriBwd));
            k_eri_sym_reduce10_ket<<<blocks_for(n - A0, 256), 256, 0, s>>>(
                n, A0, 4 * (int64_t)g.x, w.ket_part, w.jacc);
            k_eri_sym_reduce10_bra<<<blocks_for(kEriAcc * hb, 256), 256, 0, s>>>(
                n, A0, w.band, g.y, w.bra_part, w.jacc);
        }
        profile_end(kProfEriBwd, s);
        GSDFT_HIP(hipGetLastError());
        k_eri_finalize<<<blocks_for(n, 256), 256, 0, s>>>(n, 1, w.order.perm, pi, pj, w.A6,
                                                          centers, w.Nrm, w.rec, w.jacc, J,
                                                          w.contrib);
    }
    GSDFT_HIP(hipGetLastError());
    // E_J = 1/2 sum_a Pw_a J_a (gs_dft/coulomb/stream.py:319-320), fixed summation order
    GSDFT_TRY(launch_scaled_dot(n, w.q, J, 0.5, energy, w.dot_part, s));
    if (den.dP) {
        k_scatter_density_grad<<<blocks_for(n, 256), 256, 0, s>>>(n, M, pi, pj, weight, J,
                                                                  den.sym, den.dP);
        GSDFT_HIP(hipGetLastError());
    }
    if (grads) {
        k_splat_grad<<<blocks_for(M * 64, 256), 256, 0, s>>>(M, n, row_ptr, row_perm, col_ptr,
                                                             col_perm, w.contrib, quat,
                                                             log_scale, dquat, dlog_scale,
                                                             dcenters);
        GSDFT_HIP(hipGetLastError());
        if (den.dC)
            GSDFT_TRY(launch_dC(M, den.k, row_ptr, row_perm, col_ptr, col_perm, pi, pj, J,
                                weight, den.C, den.occ, den.dC, s));
    }
    return GSDFT_OK;
}

}  // namespace
}  // namespace gsdft

extern "C" int gsdft_exact_coulomb(int64_t M, const double* quat, const double* log_scale,
                                   const double* centers, int64_t k, const double* C,
                                   const double* occ, int64_t n, const int32_t* pi,
                                   const int32_t* pj, const double* weight,
                                   const int32_t* row_ptr, const int32_t* row_perm,
                                   const int32_t* col_ptr, const int32_t* col_perm,
                                   double* energy, double* J, double* dquat, double* dlog_scale,
                                   double* dcenters, double* dC, void* workspace,
                                   size_t workspace_bytes, void* stream) {
    const bool grads = dquat || dlog_scale || dcenters || dC;
    if (M <= 0 || n < 0 || k <= 0 || !C || !occ || !energy ||
        (n > 0 && (!pi || !pj || !weight || !J)))
        return fail(GSDFT_ERR_ARG, "gsdft_exact_coulomb: bad arguments");
    GSDFT_TRY(check_pairs(n, "gsdft_exact_coulomb"));
    if (grads && (!dquat || !dlog_scale || !dcenters || !dC || !row_ptr || !col_ptr ||
                  (n > 0 && (!row_perm || !col_perm))))
        return fail(GSDFT_ERR_ARG, "gsdft_exact_coulomb: the gradients come together (dquat, "
                    "dlog_scale, dcenters, dC) and need the pair index");
    const ExactDensity den{k, C, occ, nullptr, 0, dC, nullptr};
    return exact_run(M, quat, log_scale, centers, den, n, pi, pj, weight, row_ptr, row_perm,
                     col_ptr, col_perm, energy, J, dquat, dlog_scale, dcenters, grads, workspace,
                     workspace_bytes, (hipStream_t)stream, "gsdft_exact_coulomb");
}

extern "C" int gsdft_exact_coulomb_density(int64_t M, const double* quat,
                                           const double* log_scale, const double* centers,
                                           const double* P, int64_t n, const int32_t* pi,
                                           const int32_t* pj, const double* weight, int sym,
                                           const int32_t* row_ptr, const int32_t* row_perm,
                                           const int32_t* col_ptr, const int32_t* col_perm,
                                           double* energy, double* J, double* dquat,
                                           double* dlog_scale, double* dcenters, double* dP,
                                           void* workspace, size_t workspace_bytes,
                                           void* stream) {
    const bool grads = dquat || dlog_scale || dcenters;
    if (M <= 0 || n < 0 || !P || !energy || (n > 0 && (!pi || !pj || !weight || !J)))
        return fail(GSDFT_ERR_ARG, "gsdft_exact_coulomb_density: bad arguments");
    GSDFT_TRY(check_pairs(n, "gsdft_exact_coulomb_density"));
    if (M * M > (int64_t)UINT32_MAX - 255)             // dE/dP is M x M, cleared by one launch
        return fail(GSDFT_ERR_ARG, "gsdft_exact_coulomb_density: M = %lld too large for a dense "
                    "M x M dE/dP", (long long)M);
    if (grads && (!dquat || !dlog_scale || !dcenters || !row_ptr || !col_ptr ||
                  (n > 0 && (!row_perm || !col_perm))))
        return fail(GSDFT_ERR_ARG, "gsdft_exact_coulomb_density: the splat gradients come "
                    "together (dquat, dlog_scale, dcenters) and need the pair index");
    const ExactDensity den{0, nullptr, nullptr, P, sym, nullptr, dP};
    return exact_run(M, quat, log_scale, centers, den, n, pi, pj, weight, row_ptr, row_perm,
                     col_ptr, col_perm, energy, J, dquat, dlog_scale, dcenters, grads, workspace,
                     workspace_bytes, (hipStream_t)stream, "gsdft_exact_coulomb_density");
}

