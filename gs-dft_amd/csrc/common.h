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

// A quadrature table of the node integral 1/r = (2/sqrt(pi)) int_0^inf e^(-t^2 r^2) dt, passed to
// kernels by value: the 20-node half-line rule above, or, for the long-range kernel
// erf(omega r)/r = (2/sqrt(pi)) int_0^omega e^(-t^2 r^2) dt, Gauss-Legendre with kLrNodes nodes on
// [0, omega] (gs_dft/integrals/dense.py:56-76 as used by gs_dft/coulomb/ri.py:231-235).
constexpr int kLrNodes = 12;
struct NodeTable {
    double t[kNodes];
    double w[kNodes];
    int n;
};

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

// K e^-z for the quadrature node loops, z >= -1 (Tang's table-driven method): z is reduced as
// -z = (256 m + j) ln2/256 + r with |r| <= ln2/512, K e^r comes from the monic cubic
// p(r) = ((r + a2) r + a1) r + a0 (exp_cubic; K = kExpPolyK ~ 6, the node weights carry the 1/K),
// and 2^(j/256) from a 256-entry table in LDS. The cubic is the minimax fit of the relative error
// on |r| <= ln2/512 (Remez; equioscillating at 1.75e-14, evaluated in doubles within 2.0e-14 and
// unbiased, mean 4e-16): one instruction fewer than the degree-4 Taylor polynomial, whose
// 4e-17 truncation the node sums do not need (their tolerance is 1e-10 relative). Each step adds
// one scalar operand, so no coefficient has to sit in a vector register.
// z is capped at 708.3, so the result never leaves the normal range (e^-708.3 ~ 2.5e-308
// stands in for the smaller values, whose contribution to any node sum is far below round-off). A
// NaN z is lost here; callers check their inputs for NaN once per integral instead of per node.
// The integer k = 256 m + j = round(-z 256/ln2) is formed by adding 1.5 * 2^52 in the same fma:
// the sum's unit in the last place is 1, so it is rounded to an integer, which then sits in the
// low 32 bits of the mantissa as a two's-complement int (|k| <= 261581 < 2^51).
// The reduction uses ln2/256 rounded to one double (relative error d <= 2^-53) instead of a
// hi/lo pair: r then carries an absolute error ~z d, so e^-z is off by a relative z d, i.e. by
// at most z e^-z d <= 0.37 d ~ 4e-17 of the node's prefactor -- below the round-off of the sum.
// 2^m 2^(j/256) is one integer add on the high word: the table `lead` holds 2^(j/256) with j << 12
// taken off its high word (exp2_frac_lead), so adding k << 12 = (m << 20) + (j << 12) leaves
// 2^(j/256) with m added to its exponent field -- exact while the result stays normal, which the
// cap ensures (m >= -1022 and 2^(j/256) >= 1).
constexpr double kExpPolyK = 0x1.8000024e61c28p+2;     // 6.0000005498359669...
constexpr double kExpA2 = 0x1.800006265a012p+1;
constexpr double kExpA1 = 0x1.8000024e61d2cp+2;
constexpr double kExpA0 = 0x1.8000024e61bb2p+2;
// The coefficients are passed through scalar registers at every call: held in vector registers
// (where the compiler otherwise hoists them), each fma would become a register move plus an fmac.
__device__ __forceinline__ double exp_cubic(double r) {
    double a2 = kExpA2, a1 = kExpA1, a0 = kExpA0;
    asm volatile("" : "+s"(a2), "+s"(a1), "+s"(a0));
    double p = r + a2;
    p = __builtin_fma(p, r, a1);
    return __builtin_fma(p, r, a0);
}
__device__ __forceinline__ double exp_neg_tab_k(double z, const double* __restrict__ lead) {
    constexpr double kShift = 0x1.8p52;
    z = __builtin_fmin(z, 708.3);
    const double sh = __builtin_fma(z, -0x1.71547652b82fep+8, kShift);  // -z * 256/ln2 + shift
    const double kf = sh - kShift;
    const int k = (int)(uint32_t)__builtin_bit_cast(uint64_t, sh);
    const double r = __builtin_fma(-kf, 0x1.62e42fefa39efp-9, -z);      // ln2 / 256
    const double p = exp_cubic(r);
    struct Words { uint32_t lo, hi; };
    Words w = __builtin_bit_cast(Words, lead[k & 255]);
    // a 32-bit add on the high word (written out: the compiler otherwise forms a 64-bit add)
    asm("v_lshl_add_u32 %0, %1, 12, %2" : "=v"(w.hi) : "v"(k), "v"(w.hi));
    return __builtin_bit_cast(double, w) * p;
}

// The same with a node weight folded in: K wh e^-z for wh = 2^n w', where the caller passes
// z' = z - ln w' (|ln w'| <= ln2/2, so z' rounds as finely as z) and S = 1.5 * 2^52 + 256 n. The
// shift S puts k + 256 n in the low word of sh, so the high-word add scales the result by 2^n
// exactly, while sh - S is still k itself for the reduction. With n >= kFoldMinExp the cap
// kFoldCapZ keeps m + n >= -1022 (the result normal). c256 is -256/ln2 (kNegC256) held in a
// vector register by the caller (vgpr_const), so that the fma forming sh reads one scalar operand
// (S) rather than two, which would cost a register move per call.
constexpr int kFoldMinExp = -60;
constexpr double kFoldCapZ = 666.7;     // 708.3 - 60 ln 2, rounded down
constexpr double kNegC256 = -0x1.71547652b82fep+8;
__device__ __forceinline__ double vgpr_const(double c) {
    asm volatile("" : "+v"(c));
    return c;
}
__device__ __forceinline__ double exp_neg_tab_k_w(double z, double S, double c256,
                                                  const double* __restrict__ lead) {
    z = __builtin_fmin(z, kFoldCapZ);
    const double sh = __builtin_fma(z, c256, S);
    const double kf = sh - S;
    const int k = (int)(uint32_t)__builtin_bit_cast(uint64_t, sh);
    const double r = __builtin_fma(-kf, 0x1.62e42fefa39efp-9, -z);
    const double p = exp_cubic(r);
    struct Words { uint32_t lo, hi; };
    Words w = __builtin_bit_cast(Words, lead[k & 255]);
    asm("v_lshl_add_u32 %0, %1, 12, %2" : "=v"(w.hi) : "v"(k), "v"(w.hi));
    return __builtin_bit_cast(double, w) * p;
}

// Host/device split of a positive node weight for exp_neg_tab_k_w: wh = 2^n w' with n the
// nearest integer to log2 wh (at least kFoldMinExp); returns -ln w' and sets S.
__host__ __device__ inline double fold_weight(double wh, double* S) {
    int n = (int)rint(log2(wh));
    n = n < kFoldMinExp ? kFoldMinExp : n;
    *S = 0x1.8p52 + 256.0 * n;
    return -log(ldexp(wh, -n));
}

// One quadrature node in scaled form: with P = Pn(s)/s > 0 (Pn the node's determinant
// polynomial) and Q = Qn(s), so that the exponent is z = Q/P = s Qn/Pn without the product s Qn,
// returns y0 ~ P^(-1/2), ip = 1/P, zh = z - 1/2 and arg = zh - eps/2, so that
// y0 e^-arg = e^(1/2) P^(-1/2) e^-z (callers fold s^(-1/2) e^(-1/2) into the node weight); zh is
// what a reverse pass needs, s df/dPn = (f/P) zh. y0 is the hardware 1/sqrt estimate without a
// separate Newton step: its relative error is below 5.3e-8 (measured on MI355X over x in
// [1e-6, 1e8]), so |eps| < 1.1e-7 for eps = 1 - P y0^2. With h = y0^2: 1/P = h (1 + eps) +
// O(eps^2) (relative error eps^2 < 1.2e-14, which moves the node by z eps^2 e^-z <= 4.4e-15 of its
// prefactor) and P^(-1/2) = y0 e^(eps/2 + eps^2/4 + ...) (relative error eps^2/4 < 3e-15 whatever z
// is).
struct NodeValH {
    double y0;   // hardware estimate of P^(-1/2)
    double zh;   // Q / P - 1/2
    double ip;   // 1 / P
    double arg;  // zh - eps/2
};

__device__ __forceinline__ NodeValH node_val_h(double P, double Q) {
    NodeValH v;
    v.y0 = __builtin_amdgcn_rsq(P);
    const double h = v.y0 * v.y0;
    const double eps = __builtin_fma(-P, h, 1.0);
    v.ip = __builtin_fma(h, eps, h);
    v.zh = __builtin_fma(Q, v.ip, -0.5);
    v.arg = __builtin_fma(eps, -0.5, v.zh);
    return v;
}

// The forward passes need only y0 and the exponent argument: with a = Q h - 1/2,
// arg = a (1 + eps) = Q h (1 + eps) - 1/2 - eps/2, node_val_h's arg without forming 1/P.
struct NodeArgH {
    double y0;   // hardware estimate of P^(-1/2)
    double arg;  // z - 1/2 - eps/2, |eps| < 1.1e-7
};

__device__ __forceinline__ NodeArgH node_arg_h(double P, double Q) {
    NodeArgH v;
    v.y0 = __builtin_amdgcn_rsq(P);
    const double h = v.y0 * v.y0;
    const double eps = __builtin_fma(-P, h, 1.0);
    const double a = __builtin_fma(Q, h, -0.5);
    v.arg = __builtin_fma(a, eps, a);
    return v;
}

// 2^(j/256), j = 0..255, correctly rounded.
__host__ __device__ constexpr double exp2_frac(int j) {
    constexpr double t[256] = {
    0x1.0000000000000p+0, 0x1.00b1afa5abcbfp+0, 0x1.0163da9fb3335p+0, 0x1.02168143b0281p+0,
    0x1.02c9a3e778061p+0, 0x1.037d42e11bbccp+0, 0x1.04315e86e7f85p+0, 0x1.04e5f72f654b1p+0,
    0x1.059b0d3158574p+0, 0x1.0650a0e3c1f89p+0, 0x1.0706b29ddf6dep+0, 0x1.07bd42b72a836p+0,
    0x1.0874518759bc8p+0, 0x1.092bdf66607e0p+0, 0x1.09e3ecac6f383p+0, 0x1.0a9c79b1f3919p+0,
    0x1.0b5586cf9890fp+0, 0x1.0c0f145e46c85p+0, 0x1.0cc922b7247f7p+0, 0x1.0d83b23395decp+0,
    0x1.0e3ec32d3d1a2p+0, 0x1.0efa55fdfa9c5p+0, 0x1.0fb66affed31bp+0, 0x1.1073028d7233ep+0,
    0x1.11301d0125b51p+0, 0x1.11edbab5e2ab6p+0, 0x1.12abdc06c31ccp+0, 0x1.136a814f204abp+0,
    0x1.1429aaea92de0p+0, 0x1.14e95934f312ep+0, 0x1.15a98c8a58e51p+0, 0x1.166a45471c3c2p+0,
    0x1.172b83c7d517bp+0, 0x1.17ed48695bbc0p+0, 0x1.18af9388c8deap+0, 0x1.1972658375d2fp+0,
    0x1.1a35beb6fcb75p+0, 0x1.1af99f8138a1cp+0, 0x1.1bbe084045cd4p+0, 0x1.1c82f95281c6bp+0,
    0x1.1d4873168b9aap+0, 0x1.1e0e75eb44027p+0, 0x1.1ed5022fcd91dp+0, 0x1.1f9c18438ce4dp+0,
    0x1.2063b88628cd6p+0, 0x1.212be3578a819p+0, 0x1.21f49917ddc96p+0, 0x1.22bdda27912d1p+0,
    0x1.2387a6e756238p+0, 0x1.2451ffb82140ap+0, 0x1.251ce4fb2a63fp+0, 0x1.25e85711ece75p+0,
    0x1.26b4565e27cddp+0, 0x1.2780e341ddf29p+0, 0x1.284dfe1f56381p+0, 0x1.291ba7591bb70p+0,
    0x1.29e9df51fdee1p+0, 0x1.2ab8a66d10f13p+0, 0x1.2b87fd0dad990p+0, 0x1.2c57e39771b2fp+0,
    0x1.2d285a6e4030bp+0, 0x1.2df961f641589p+0, 0x1.2ecafa93e2f56p+0, 0x1.2f9d24abd886bp+0,
    0x1.306fe0a31b715p+0, 0x1.31432edeeb2fdp+0, 0x1.32170fc4cd831p+0, 0x1.32eb83ba8ea32p+0,
    0x1.33c08b26416ffp+0, 0x1.3496266e3fa2dp+0, 0x1.356c55f929ff1p+0, 0x1.36431a2de883bp+0,
    0x1.371a7373aa9cbp+0, 0x1.37f26231e754ap+0, 0x1.38cae6d05d866p+0, 0x1.39a401b7140efp+0,
    0x1.3a7db34e59ff7p+0, 0x1.3b57fbfec6cf4p+0, 0x1.3c32dc313a8e5p+0, 0x1.3d0e544ede173p+0,
    0x1.3dea64c123422p+0, 0x1.3ec70df1c5175p+0, 0x1.3fa4504ac801cp+0, 0x1.40822c367a024p+0,
    0x1.4160a21f72e2ap+0, 0x1.423fb2709468ap+0, 0x1.431f5d950a897p+0, 0x1.43ffa3f84b9d4p+0,
    0x1.44e086061892dp+0, 0x1.45c2042a7d232p+0, 0x1.46a41ed1d0057p+0, 0x1.4786d668b3237p+0,
    0x1.486a2b5c13cd0p+0, 0x1.494e1e192aed2p+0, 0x1.4a32af0d7d3dep+0, 0x1.4b17dea6db7d7p+0,
    0x1.4bfdad5362a27p+0, 0x1.4ce41b817c114p+0, 0x1.4dcb299fddd0dp+0, 0x1.4eb2d81d8abffp+0,
    0x1.4f9b2769d2ca7p+0, 0x1.508417f4531eep+0, 0x1.516daa2cf6642p+0, 0x1.5257de83f4eefp+0,
    0x1.5342b569d4f82p+0, 0x1.542e2f4f6ad27p+0, 0x1.551a4ca5d920fp+0, 0x1.56070dde910d2p+0,
    0x1.56f4736b527dap+0, 0x1.57e27dbe2c4cfp+0, 0x1.58d12d497c7fdp+0, 0x1.59c0827ff07ccp+0,
    0x1.5ab07dd485429p+0, 0x1.5ba11fba87a03p+0, 0x1.5c9268a5946b7p+0, 0x1.5d84590998b93p+0,
    0x1.5e76f15ad2148p+0, 0x1.5f6a320dceb71p+0, 0x1.605e1b976dc09p+0, 0x1.6152ae6cdf6f4p+0,
    0x1.6247eb03a5585p+0, 0x1.633dd1d1929fdp+0, 0x1.6434634ccc320p+0, 0x1.652b9febc8fb7p+0,
    0x1.6623882552225p+0, 0x1.671c1c70833f6p+0, 0x1.68155d44ca973p+0, 0x1.690f4b19e9538p+0,
    0x1.6a09e667f3bcdp+0, 0x1.6b052fa75173ep+0, 0x1.6c012750bdabfp+0, 0x1.6cfdcddd47645p+0,
    0x1.6dfb23c651a2fp+0, 0x1.6ef9298593ae5p+0, 0x1.6ff7df9519484p+0, 0x1.70f7466f42e87p+0,
    0x1.71f75e8ec5f74p+0, 0x1.72f8286ead08ap+0, 0x1.73f9a48a58174p+0, 0x1.74fbd35d7cbfdp+0,
    0x1.75feb564267c9p+0, 0x1.77024b1ab6e09p+0, 0x1.780694fde5d3fp+0, 0x1.790b938ac1cf6p+0,
    0x1.7a11473eb0187p+0, 0x1.7b17b0976cfdbp+0, 0x1.7c1ed0130c132p+0, 0x1.7d26a62ff86f0p+0,
    0x1.7e2f336cf4e62p+0, 0x1.7f3878491c491p+0, 0x1.80427543e1a12p+0, 0x1.814d2add106d9p+0,
    0x1.82589994cce13p+0, 0x1.8364c1eb941f7p+0, 0x1.8471a4623c7adp+0, 0x1.857f4179f5b21p+0,
    0x1.868d99b4492edp+0, 0x1.879cad931a436p+0, 0x1.88ac7d98a6699p+0, 0x1.89bd0a478580fp+0,
    0x1.8ace5422aa0dbp+0, 0x1.8be05bad61778p+0, 0x1.8cf3216b5448cp+0, 0x1.8e06a5e0866d9p+0,
    0x1.8f1ae99157736p+0, 0x1.902fed0282c8ap+0, 0x1.9145b0b91ffc6p+0, 0x1.925c353aa2fe2p+0,
    0x1.93737b0cdc5e5p+0, 0x1.948b82b5f98e5p+0, 0x1.95a44cbc8520fp+0, 0x1.96bdd9a7670b3p+0,
    0x1.97d829fde4e50p+0, 0x1.98f33e47a22a2p+0, 0x1.9a0f170ca07bap+0, 0x1.9b2bb4d53fe0dp+0,
    0x1.9c49182a3f090p+0, 0x1.9d674194bb8d5p+0, 0x1.9e86319e32323p+0, 0x1.9fa5e8d07f29ep+0,
    0x1.a0c667b5de565p+0, 0x1.a1e7aed8eb8bbp+0, 0x1.a309bec4a2d33p+0, 0x1.a42c980460ad8p+0,
    0x1.a5503b23e255dp+0, 0x1.a674a8af46052p+0, 0x1.a799e1330b358p+0, 0x1.a8bfe53c12e59p+0,
    0x1.a9e6b5579fdbfp+0, 0x1.ab0e521356ebap+0, 0x1.ac36bbfd3f37ap+0, 0x1.ad5ff3a3c2774p+0,
    0x1.ae89f995ad3adp+0, 0x1.afb4ce622f2ffp+0, 0x1.b0e07298db666p+0, 0x1.b20ce6c9a8952p+0,
    0x1.b33a2b84f15fbp+0, 0x1.b468415b749b1p+0, 0x1.b59728de5593ap+0, 0x1.b6c6e29f1c52ap+0,
    0x1.b7f76f2fb5e47p+0, 0x1.b928cf22749e4p+0, 0x1.ba5b030a1064ap+0, 0x1.bb8e0b79a6f1fp+0,
    0x1.bcc1e904bc1d2p+0, 0x1.bdf69c3f3a207p+0, 0x1.bf2c25bd71e09p+0, 0x1.c06286141b33dp+0,
    0x1.c199bdd85529cp+0, 0x1.c2d1cd9fa652cp+0, 0x1.c40ab5fffd07ap+0, 0x1.c544778fafb22p+0,
    0x1.c67f12e57d14bp+0, 0x1.c7ba88988c933p+0, 0x1.c8f6d9406e7b5p+0, 0x1.ca3405751c4dbp+0,
    0x1.cb720dcef9069p+0, 0x1.ccb0f2e6d1675p+0, 0x1.cdf0b555dc3fap+0, 0x1.cf3155b5bab74p+0,
    0x1.d072d4a07897cp+0, 0x1.d1b532b08c968p+0, 0x1.d2f87080d89f2p+0, 0x1.d43c8eacaa1d6p+0,
    0x1.d5818dcfba487p+0, 0x1.d6c76e862e6d3p+0, 0x1.d80e316c98398p+0, 0x1.d955d71ff6075p+0,
    0x1.da9e603db3285p+0, 0x1.dbe7cd63a8315p+0, 0x1.dd321f301b460p+0, 0x1.de7d5641c0658p+0,
    0x1.dfc97337b9b5fp+0, 0x1.e11676b197d17p+0, 0x1.e264614f5a129p+0, 0x1.e3b333b16ee12p+0,
    0x1.e502ee78b3ff6p+0, 0x1.e653924676d76p+0, 0x1.e7a51fbc74c83p+0, 0x1.e8f7977cdb740p+0,
    0x1.ea4afa2a490dap+0, 0x1.eb9f4867cca6ep+0, 0x1.ecf482d8e67f1p+0, 0x1.ee4aaa2188510p+0,
    0x1.efa1bee615a27p+0, 0x1.f0f9c1cb6412ap+0, 0x1.f252b376bba97p+0, 0x1.f3ac948dd7274p+0,
    0x1.f50765b6e4540p+0, 0x1.f6632798844f8p+0, 0x1.f7bfdad9cbe14p+0, 0x1.f91d802243c89p+0,
    0x1.fa7c1819e90d8p+0, 0x1.fbdba3692d514p+0, 0x1.fd3c22b8f71f1p+0, 0x1.fe9d96b2a23d9p+0,
    };
    return t[j];
}

// exp2_frac(j) with j << 12 taken off its high word (the table of exp_neg_tab_k).
__host__ __device__ inline double exp2_frac_lead(int j) {
    return __builtin_bit_cast(double, __builtin_bit_cast(uint64_t, exp2_frac(j)) -
                                          ((uint64_t)j << 44));
}

// 1/sqrt(x) for positive normal x: the hardware estimate (relative error ~5e-8) refined by one
// Newton step y <- y + y (1 - x y^2) / 2 (relative error < 5e-15).
__device__ __forceinline__ double rsqrt1(double x) {
    const double y = __builtin_amdgcn_rsq(x);
    const double e = __builtin_fma(-x * y, y, 1.0);
    return __builtin_fma(y * 0.5, e, y);
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

// Reverse of the chart for splat m: from acc = dE/dA (six slots, dE = sum over all nine entries),
// dE/dmu (3) and dE/dN (1) to dE/dquat, dE/dlog_scale and dE/dcenters
// (gs_dft/basis/spectral.py:33-40,72-82 under JAX autodiff).
__device__ inline void chart_reverse(int64_t m, const double acc[10],
                                     const double* __restrict__ quat,
                                     const double* __restrict__ log_scale,
                                     double* __restrict__ dquat, double* __restrict__ dlog_scale,
                                     double* __restrict__ dcenters) {
    const double* q = quat + 4 * m;
    const double* l = log_scale + 3 * m;
    double R[9], qn[4], nrm;
    quat_rotation(q, R, qn, &nrm);
    const double av[3] = {exp(l[0]), exp(l[1]), exp(l[2])};
    const double Nm = pow(8.0 * exp(l[0] + l[1] + l[2]) / kPi3, 0.25);
    const double G[9] = {acc[0], acc[3], acc[4], acc[3], acc[1], acc[5], acc[4], acc[5], acc[2]};
    double GR[9];
    for (int r = 0; r < 3; ++r)
        for (int c = 0; c < 3; ++c)
            GR[3 * r + c] = G[3 * r] * R[c] + G[3 * r + 1] * R[3 + c] + G[3 * r + 2] * R[6 + c];
    for (int jx = 0; jx < 3; ++jx) {
        const double ga = R[jx] * GR[jx] + R[3 + jx] * GR[3 + jx] + R[6 + jx] * GR[6 + jx];
        dlog_scale[3 * m + jx] = av[jx] * ga + acc[9] * Nm * 0.25;
    }
    double gR[9];
    for (int r = 0; r < 3; ++r)
        for (int c = 0; c < 3; ++c) gR[3 * r + c] = 2.0 * av[c] * GR[3 * r + c];
    const double w = qn[0], x = qn[1], yq = qn[2], z = qn[3];
    const double gqn[4] = {
        2 * (-z * gR[1] + yq * gR[2] + z * gR[3] - x * gR[5] - yq * gR[6] + x * gR[7]),
        2 * (yq * gR[1] + z * gR[2] + yq * gR[3] - 2 * x * gR[4] - w * gR[5] + z * gR[6]
             + w * gR[7] - 2 * x * gR[8]),
        2 * (-2 * yq * gR[0] + x * gR[1] + w * gR[2] + x * gR[3] + z * gR[5] - w * gR[6]
             + z * gR[7] - 2 * yq * gR[8]),
        2 * (-2 * z * gR[0] - w * gR[1] + x * gR[2] + w * gR[3] - 2 * z * gR[4] + yq * gR[5]
             + x * gR[6] + yq * gR[7])};
    const double den = nrm + 1e-12;
    const double dot = q[0] * gqn[0] + q[1] * gqn[1] + q[2] * gqn[2] + q[3] * gqn[3];
    for (int t = 0; t < 4; ++t) dquat[4 * m + t] = gqn[t] / den - q[t] * dot / (nrm * den * den);
    for (int t = 0; t < 3; ++t) dcenters[3 * m + t] = acc[6 + t];
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
// v broadcast from one lane (wave-uniform lane index) to the whole wave.
__device__ __forceinline__ double readlane_f64(double v, int lane) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), lane);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ double wave_sum(double v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Centre-grouped slot order of a product aux of G = N / M exponent scales (scale-major,
// P = s M + m): slot m G + s, so the scales sharing a centre are consecutive; G <= 1 keeps aux
// order.
__host__ __device__ __forceinline__ int64_t aux_slot(int64_t p, int64_t N, int64_t G) {
    if (G <= 1) return p;
    const int64_t Mg = N / G;
    return (p % Mg) * G + p / Mg;
}

__host__ __device__ __forceinline__ int64_t aux_of_slot(int64_t q, int64_t N, int64_t G) {
    if (G <= 1) return q;
    const int64_t Mg = N / G;
    return (q % G) * Mg + q / G;
}

}  // namespace gsdft
