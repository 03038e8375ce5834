// Shared device helpers for the DF-J library (gfx950, FP64 throughout).
//
// Storage conventions:
//   * per-splat precision A is symmetric and held as 6 doubles: xx, yy, zz, xy, xz, yz;
//   * symmetric gradient matrices use the same 6 slots, with dE = sum_kl G_kl dA_kl over all nine
//     entries (so an off-diagonal slot carries G_kl = G_lk, not their sum);
//   * every N x N matrix is row-major.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gsdft {

// Constants exactly as the reference evaluates them in Python floats.
constexpr double kPi = 0x1.921fb54442d18p+1;        // math.pi
constexpr double kPi3 = 0x1.f019b59389d7bp+4;       // math.pi ** 3
constexpr double kPi15 = 0x1.645f7c63f2c6bp+2;      // math.pi ** 1.5
constexpr double kTwoPi25 = 0x1.17e50a9dc6553p+5;   // 2.0 * math.pi ** 2.5
constexpr double kPref3c = 0x1.17e50a9dc6553p+5;    // 2.0 * math.pi ** 3 / math.sqrt(math.pi)

constexpr int kNodes = 20;

// 20-node Gauss-Legendre on [0, inf) via t = s/(1-s): numpy.polynomial.legendre.leggauss(20)
// mapped as gs_dft/integrals/dense.py:46-53 does, stored bit-exactly.
__host__ __device__ constexpr double quad_t(int i) {
    constexpr double t[kNodes] = {
        0x1.c3e06b40c0727p-9, 0x1.2c8e6342a4a5ep-6, 0x1.77fcb58d6ada9p-5, 0x1.664fc2d4e4d91p-4,
        0x1.297cd9a7af59bp-3, 0x1.c795d86bbc171p-3, 0x1.4b8359ef99024p-2, 0x1.d2db83eb796e2p-2,
        0x1.42058bd8ac113p-1, 0x1.b7351894990f0p-1, 0x1.2a6db1103b037p+0, 0x1.97074cba11770p+0,
        0x1.18c0f758aca43p+1, 0x1.8b60024c1b4f7p+1, 0x1.1fb3418486a0fp+2, 0x1.b898abea34f68p+2,
        0x1.6dcdf6bbc2279p+3, 0x1.5c9b8fcc0a6fap+4, 0x1.b4191f8d04cd7p+5, 0x1.220fbc4965a88p+8};
    return t[i];
}
__host__ __device__ constexpr double quad_w(int i) {
    constexpr double w[kNodes] = {
        0x1.2294c7120a5a9p-7, 0x1.58ebfe9762aa7p-6, 0x1.18cf317b25b59p-5, 0x1.9363ccbfca34ep-5,
        0x1.11cdae4285cf3p-4, 0x1.69bc85b3fc938p-4, 0x1.d89763771433ep-4, 0x1.346db18e63689p-3,
        0x1.95538e7c056a5p-3, 0x1.0df14a79d44aep-2, 0x1.6ed603ef2a5e2p-2, 0x1.002975fc1d907p-1,
        0x1.72f578bf3121dp-1, 0x1.19d0adfafd239p+0, 0x1.c8debb31e0867p+0, 0x1.9584c4e1f7391p+1,
        0x1.9bd353a94748bp+2, 0x1.045c595b5d172p+4, 0x1.f478ac84cc948p+5, 0x1.750cec4d183bdp+9};
    return w[i];
}

// ------------------------------------------------------------------ fast FP64 transcendentals
// e^x by Cody-Waite reduction x = k ln2 + r, |r| <= ln2/2, and the degree-12 Taylor polynomial of
// e^r in Horner form (truncation < 2e-16 relative), rescaled by ldexp. ln2 is split into the
// classic fdlibm hi/lo pair so k*ln2_hi is exact. Below -746 the result is 0; NaN propagates.
__device__ __forceinline__ double exp_fast(double x) {
    x = (x < -746.0) ? -746.0 : x;
    const double kf = __builtin_rint(x * 0x1.71547652b82fep+0);        // x / ln 2
    double r = __builtin_fma(-kf, 0x1.62e42fee00000p-1, x);            // ln2_hi
    r = __builtin_fma(-kf, 0x1.a39ef35793c76p-33, r);                  // ln2_lo
    double p = 2.08767569878680989792e-09;                             // 1/12!
    p = __builtin_fma(p, r, 2.50521083854417187751e-08);               // 1/11!
    p = __builtin_fma(p, r, 2.75573192239858906526e-07);               // 1/10!
    p = __builtin_fma(p, r, 2.75573192239858906526e-06);               // 1/9!
    p = __builtin_fma(p, r, 2.48015873015873015873e-05);               // 1/8!
    p = __builtin_fma(p, r, 1.98412698412698412698e-04);               // 1/7!
    p = __builtin_fma(p, r, 1.38888888888888888889e-03);               // 1/6!
    p = __builtin_fma(p, r, 8.33333333333333333333e-03);               // 1/5!
    p = __builtin_fma(p, r, 4.16666666666666666667e-02);               // 1/4!
    p = __builtin_fma(p, r, 1.66666666666666666667e-01);               // 1/3!
    p = __builtin_fma(p, r, 0.5);
    p = __builtin_fma(p, r, 1.0);
    p = __builtin_fma(p, r, 1.0);
    return __builtin_ldexp(p, (int)kf);
}

// 1/sqrt(x) for positive normal x: the hardware estimate refined by two Newton steps
// y <- y + y (1 - x y^2) / 2.
__device__ __forceinline__ double rsqrt_nr(double x) {
    double y = __builtin_amdgcn_rsq(x);
    double e = __builtin_fma(-x * y, y, 1.0);
    y = __builtin_fma(y * 0.5, e, y);
    e = __builtin_fma(-x * y, y, 1.0);
    y = __builtin_fma(y * 0.5, e, y);
    return y;
}

// ------------------------------------------------------------------ 3x3 symmetric algebra
// The nine-entry forms below follow gs_dft/integrals/linalg3.py:17-51 term by term, reading the
// symmetric matrix through its six slots. S(r,c) maps a (row, col) to the slot.
struct Sym3 {
    double xx, yy, zz, xy, xz, yz;
    __host__ __device__ double at(int r, int c) const {
        if (r == c) return r == 0 ? xx : (r == 1 ? yy : zz);
        int s = r + c;                       // 1: xy, 2: xz, 3: yz
        return s == 1 ? xy : (s == 2 ? xz : yz);
    }
};

__device__ __forceinline__ Sym3 load_sym(const double* __restrict__ p) {
    return Sym3{p[0], p[1], p[2], p[3], p[4], p[5]};
}

// gs_dft/integrals/linalg3.py:17-22 (cofactor expansion along the first row).
__device__ __forceinline__ double det3(const Sym3& A) {
    return A.xx * (A.yy * A.zz - A.yz * A.yz)
         - A.xy * (A.xy * A.zz - A.yz * A.xz)
         + A.xz * (A.xy * A.yz - A.yy * A.xz);
}

// gs_dft/integrals/linalg3.py:26-41, full 3x3 adjugate c[r][c] of a symmetric A.
__device__ __forceinline__ void adj3(const Sym3& A, double c[9]) {
    c[0] = A.yy * A.zz - A.yz * A.yz;
    c[1] = A.xz * A.yz - A.xy * A.zz;
    c[2] = A.xy * A.yz - A.xz * A.yy;
    c[3] = A.yz * A.xz - A.xy * A.zz;
    c[4] = A.xx * A.zz - A.xz * A.xz;
    c[5] = A.xz * A.xy - A.xx * A.yz;
    c[6] = A.xy * A.yz - A.yy * A.xz;
    c[7] = A.xy * A.xz - A.xx * A.yz;
    c[8] = A.xx * A.yy - A.xy * A.xy;
}

__device__ __forceinline__ void matvec(const Sym3& A, const double x[3], double y[3]) {
    y[0] = A.xx * x[0] + A.xy * x[1] + A.xz * x[2];
    y[1] = A.xy * x[0] + A.yy * x[1] + A.yz * x[2];
    y[2] = A.xz * x[0] + A.yz * x[1] + A.zz * x[2];
}

// gs_dft/integrals/linalg3.py:49-51: adj(A) b / det(A).
__device__ __forceinline__ void solve3(const Sym3& A, const double b[3], double x[3]) {
    double c[9];
    adj3(A, c);
    const double det = det3(A);
    x[0] = (c[0] * b[0] + c[1] * b[1] + c[2] * b[2]) / det;
    x[1] = (c[3] * b[0] + c[4] * b[1] + c[5] * b[2]) / det;
    x[2] = (c[6] * b[0] + c[7] * b[1] + c[8] * b[2]) / det;
}

__device__ __forceinline__ Sym3 add(const Sym3& a, const Sym3& b) {
    return Sym3{a.xx + b.xx, a.yy + b.yy, a.zz + b.zz, a.xy + b.xy, a.xz + b.xz, a.yz + b.yz};
}

// G += s * sym(x y^T), the gradient matrix of s * x^T dA y for a symmetric dA.
__device__ __forceinline__ void add_sym_outer(double G[6], double s, const double x[3],
                                              const double y[3]) {
    G[0] += s * (x[0] * y[0]);
    G[1] += s * (x[1] * y[1]);
    G[2] += s * (x[2] * y[2]);
    G[3] += 0.5 * s * (x[0] * y[1] + y[0] * x[1]);
    G[4] += 0.5 * s * (x[0] * y[2] + y[0] * x[2]);
    G[5] += 0.5 * s * (x[1] * y[2] + y[1] * x[2]);
}

// ------------------------------------------------------------------ chart
// gs_dft/basis/spectral.py:33-40. Returns the rotation of the normalised quaternion.
__device__ __forceinline__ void quat_rotation(const double* __restrict__ q, double R[9],
                                              double qn[4], double* nrm_out) {
    const double nrm = sqrt(q[0] * q[0] + q[1] * q[1] + q[2] * q[2] + q[3] * q[3]);
    const double den = nrm + 1e-12;
    const double w = q[0] / den, x = q[1] / den, y = q[2] / den, z = q[3] / den;
    R[0] = 1 - 2 * (y * y + z * z); R[1] = 2 * (x * y - w * z); R[2] = 2 * (x * z + w * y);
    R[3] = 2 * (x * y + w * z); R[4] = 1 - 2 * (x * x + z * z); R[5] = 2 * (y * z - w * x);
    R[6] = 2 * (x * z - w * y); R[7] = 2 * (y * z + w * x); R[8] = 1 - 2 * (x * x + y * y);
    qn[0] = w; qn[1] = x; qn[2] = y; qn[3] = z;
    *nrm_out = nrm;
}

// gs_dft/basis/spectral.py:72-82: A = R diag(e^l) R^T (entry ik = sum_j (R_ij a_j) R_kj, upper
// triangle evaluated and mirrored) and N = (8 det A / pi^3)^(1/4), det A = e^(l0+l1+l2).
__device__ __forceinline__ void splat_chart(const double* __restrict__ q,
                                            const double* __restrict__ l, Sym3* A, double* N) {
    double R[9], qn[4], nrm;
    quat_rotation(q, R, qn, &nrm);
    const double a0 = exp(l[0]), a1 = exp(l[1]), a2 = exp(l[2]);
    auto ent = [&](int i, int k) {
        return (R[3 * i] * a0) * R[3 * k] + (R[3 * i + 1] * a1) * R[3 * k + 1]
             + (R[3 * i + 2] * a2) * R[3 * k + 2];
    };
    *A = Sym3{ent(0, 0), ent(1, 1), ent(2, 2), ent(0, 1), ent(0, 2), ent(1, 2)};
    *N = pow(8.0 * exp(l[0] + l[1] + l[2]) / kPi3, 0.25);
}

// ------------------------------------------------------------------ pair quantities
// gs_dft/coulomb/stream.py:203-215: Ah = Ai + Aj, P = Ah^-1 (Ai mu_i + Aj mu_j),
// KN = N_i N_j exp(-d . Ai Ah^-1 Aj d), d = mu_i - mu_j.
__device__ __forceinline__ void pair_quantities(const Sym3& Ai, const Sym3& Aj,
                                                const double mui[3], const double muj[3],
                                                double Ni, double Nj, Sym3* Ah, double P[3],
                                                double* KN) {
    *Ah = add(Ai, Aj);
    double r1[3], r2[3], rhs[3];
    matvec(Ai, mui, r1);
    matvec(Aj, muj, r2);
    rhs[0] = r1[0] + r2[0]; rhs[1] = r1[1] + r2[1]; rhs[2] = r1[2] + r2[2];
    solve3(*Ah, rhs, P);
    const double d[3] = {mui[0] - muj[0], mui[1] - muj[1], mui[2] - muj[2]};
    double Ajd[3], x[3], z[3];
    matvec(Aj, d, Ajd);
    solve3(*Ah, Ajd, x);
    matvec(Ai, x, z);
    const double e = d[0] * z[0] + d[1] * z[1] + d[2] * z[2];
    *KN = Ni * Nj * exp(-e);
}

// ------------------------------------------------------------------ wave helpers
__device__ __forceinline__ double wave_sum(double v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

}  // namespace gsdft
