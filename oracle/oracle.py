"""numpy bindings of the C oracle (``oracle/c/oracle.c``).

TEST INFRASTRUCTURE ONLY: the parity checker for the HIP path and the benchmark's CPU baseline.
The shipped package never imports this module.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
import pathlib
import subprocess

import numpy as np

_HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = _HERE / "build" / "liboracle.so"

_lib = None

_D = ctypes.POINTER(ctypes.c_double)
_I32 = ctypes.POINTER(ctypes.c_int32)
_I64 = ctypes.POINTER(ctypes.c_int64)
_i64 = ctypes.c_int64


def build() -> pathlib.Path:
    """Compile the oracle with its Makefile (gcc + OpenMP)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        L.orc_count_significant.restype = ctypes.c_int64
        L.orc_boys0.restype = ctypes.c_double
        L.orc_boys0.argtypes = [ctypes.c_double]
        L.orc_neighbor_pairs.restype = ctypes.c_int
        L.orc_cholesky.restype = ctypes.c_int
        L.orc_num_threads.restype = ctypes.c_int
        L.orc_external_energy.restype = ctypes.c_double
        L.orc_exact_coulomb.restype = ctypes.c_double
        # the reference's own table (gs_dft/integrals/dense.py:46-53, numpy leggauss)
        t, w = reference_quad_table(20)
        L.orc_set_quad_table(_d(t), _d(w))
        _lib = L
    return _lib


def _d(a):
    return a.ctypes.data_as(_D)


def _f64(a):
    return np.ascontiguousarray(a, dtype=np.float64)


def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


def reference_quad_table(n: int = 20):
    """gs_dft/integrals/dense.py:46-53: numpy leggauss mapped to [0, inf) by t = s/(1-s)."""
    x, wl = np.polynomial.legendre.leggauss(n)
    s = (x + 1.0) / 2.0
    t = np.ascontiguousarray(s / (1.0 - s), dtype=np.float64)
    w = np.ascontiguousarray((wl / 2.0) * (1.0 / (1.0 - s) ** 2), dtype=np.float64)
    return t, w


def lr_quad_table(omega: float, n: int = 12):
    """gs_dft/integrals/dense.py:56-76 (_gauss_legendre_segment, as ri.py:231-235 calls it):
    numpy leggauss(n) mapped to [0, omega], the rule of the long-range kernel erf(omega r)/r."""
    x, wl = np.polynomial.legendre.leggauss(n)
    t = np.ascontiguousarray(0.5 * float(omega) * (x + 1.0), dtype=np.float64)
    w = np.ascontiguousarray(0.5 * float(omega) * wl, dtype=np.float64)
    return t, w


@contextlib.contextmanager
def node_rule(t, w):
    """Every three-centre routine integrates with the rule (t, w) (at most 20 nodes) inside the
    block: the table is padded with zero-weight nodes at t = 0, which add exactly 0 to every node
    sum and its derivatives; the reference's 20-node table is restored on exit."""
    t, w = np.asarray(t, dtype=np.float64), np.asarray(w, dtype=np.float64)
    if t.shape != w.shape or t.ndim != 1 or len(t) > 20:
        raise ValueError("node_rule: t and w must be 1-D of the same length <= 20")
    tp, wp = np.zeros(20), np.zeros(20)
    tp[:len(t)], wp[:len(w)] = t, w
    L = lib()
    L.orc_set_quad_table(_d(tp), _d(wp))
    try:
        yield
    finally:
        tr, wr = reference_quad_table(20)
        L.orc_set_quad_table(_d(tr), _d(wr))


def num_threads() -> int:
    return int(lib().orc_num_threads())


def quad_table(n: int = 20):
    t = np.empty(n)
    w = np.empty(n)
    lib().orc_quad_table(ctypes.c_int(n), _d(t), _d(w))
    return t, w


def chart(quat, log_scale):
    quat, log_scale = _f64(quat), _f64(log_scale)
    M = quat.shape[0]
    A = np.empty((M, 3, 3))
    N = np.empty(M)
    lib().orc_chart(_i64(M), _d(quat), _d(log_scale), _d(A), _d(N))
    return A, N


def pair_quantities(A, mu, norm, pi, pj):
    A, mu, norm, pi, pj = _f64(A), _f64(mu), _f64(norm), _i32(pi), _i32(pj)
    n = pi.shape[0]
    Ah = np.empty((n, 3, 3))
    P = np.empty((n, 3))
    KN = np.empty(n)
    lib().orc_pair_quantities(_i64(A.shape[0]), _d(A), _d(mu), _d(norm), _i64(n),
                              pi.ctypes.data_as(_I32), pj.ctypes.data_as(_I32),
                              _d(Ah), _d(P), _d(KN))
    return Ah, P, KN


def overlap_pairs(quat, log_scale, centers, pi, pj):
    quat, log_scale, centers, pi, pj = _f64(quat), _f64(log_scale), _f64(centers), _i32(pi), _i32(pj)
    S = np.empty(pi.shape[0])
    lib().orc_overlap_pairs(_i64(quat.shape[0]), _d(quat), _d(log_scale), _d(centers),
                            _i64(pi.shape[0]), pi.ctypes.data_as(_I32), pj.ctypes.data_as(_I32),
                            _d(S))
    return S


def count_significant(quat, log_scale, centers, eps, unique):
    quat, log_scale, centers = _f64(quat), _f64(log_scale), _f64(centers)
    return int(lib().orc_count_significant(_i64(quat.shape[0]), _d(quat), _d(log_scale),
                                           _d(centers), ctypes.c_double(eps), ctypes.c_int(int(unique))))


def neighbor_pairs(quat, log_scale, centers, eps, pad_to=None, unique=False):
    """(pi, pj, weight, n_sig). Raises ValueError where the reference raises (n_sig > 2 pad)."""
    quat, log_scale, centers = _f64(quat), _f64(log_scale), _f64(centers)
    M = quat.shape[0]
    n_all = M * (M + 1) // 2 if unique else M * M
    if pad_to is None:
        length = n_all if eps < 0 else count_significant(quat, log_scale, centers, eps, unique)
    else:
        length = int(pad_to)
    pi = np.zeros(max(length, 1), np.int32)
    pj = np.zeros(max(length, 1), np.int32)
    w = np.zeros(max(length, 1))
    n_out = ctypes.c_int64()
    n_sig = ctypes.c_int64()
    rc = lib().orc_neighbor_pairs(_i64(M), _d(quat), _d(log_scale), _d(centers),
                                  ctypes.c_double(eps), _i64(-1 if pad_to is None else int(pad_to)),
                                  ctypes.c_int(int(unique)), pi.ctypes.data_as(_I32),
                                  pj.ctypes.data_as(_I32), _d(w), ctypes.byref(n_out),
                                  ctypes.byref(n_sig))
    if rc == 2:
        raise ValueError(f"neighbor_pairs: {n_sig.value} significant pairs exceed 2x the pad "
                         f"({2 * int(pad_to)})")
    m = int(n_out.value)
    return pi[:m], pj[:m], w[:m], int(n_sig.value)


def screen_margin(quat, log_scale, centers, eps, unique, rel_tol=1e-10):
    """(number of candidates with ||S| - eps| <= rel_tol eps, min ||S| - eps| / eps)."""
    quat, log_scale, centers = _f64(quat), _f64(log_scale), _f64(centers)
    n_close = ctypes.c_int64()
    gap = ctypes.c_double()
    lib().orc_screen_margin(_i64(quat.shape[0]), _d(quat), _d(log_scale), _d(centers),
                            ctypes.c_double(eps), ctypes.c_int(int(unique)),
                            ctypes.c_double(rel_tol), ctypes.byref(n_close), ctypes.byref(gap))
    return int(n_close.value), float(gap.value)


def spatial_audit(quat, log_scale, centers, eps, unique, safety=1.25):
    """Brute-force check of the spatial candidate rules (gs_dft/screening/pairs.py:167-197):
    dict with the significant count, each rule's candidate count and the significant pairs it
    misses, and the largest |d|^2 / (L (1/lmin_i + 1/lmin_j)) over the significant pairs."""
    quat, log_scale, centers = _f64(quat), _f64(log_scale), _f64(centers)
    out = [ctypes.c_int64() for _ in range(5)]
    mx = ctypes.c_double()
    lib().orc_spatial_audit(_i64(quat.shape[0]), _d(quat), _d(log_scale), _d(centers),
                            ctypes.c_double(eps), ctypes.c_int(int(unique)),
                            ctypes.c_double(safety), *(ctypes.byref(o) for o in out),
                            ctypes.byref(mx))
    keys = ("n_sig", "n_cand_ref", "n_miss_ref", "n_cand_bound", "n_miss_bound")
    r = {k: int(o.value) for k, o in zip(keys, out)}
    r["max_ratio"] = float(mx.value)
    return r


def product_aux(quat, log_scale, centers, scales):
    quat, log_scale, centers = _f64(quat), _f64(log_scale), _f64(centers)
    sc = _f64(np.asarray(scales, float))
    M = quat.shape[0]
    la = np.empty(len(sc) * M)
    cen = np.empty((len(sc) * M, 3))
    lib().orc_product_aux(_i64(M), _d(quat), _d(log_scale), _d(centers), _d(sc),
                          ctypes.c_int(len(sc)), _d(la), _d(cen))
    return la, cen


def product_aux_pairs(quat, log_scale, centers, pi, pj, valid, scales):
    """Product aux of the listed pairs (gs_dft/basis/isotropic.py:106-116, diagonal_only=False):
    (log_alpha (S*n,), centres (S*n, 3)), scale-major; ``valid`` None or per-entry weights."""
    quat, log_scale, centers = _f64(quat), _f64(log_scale), _f64(centers)
    pi, pj = _i32(pi), _i32(pj)
    v = None if valid is None else _f64(np.asarray(valid, dtype=np.float64))
    sc = _f64(np.asarray(scales, float))
    n = pi.shape[0]
    la = np.empty(len(sc) * n)
    cen = np.empty((len(sc) * n, 3))
    lib().orc_product_aux_pairs(_i64(quat.shape[0]), _d(quat), _d(log_scale), _d(centers),
                                _i64(n), pi.ctypes.data_as(_I32), pj.ctypes.data_as(_I32),
                                None if v is None else _d(v), _d(sc), ctypes.c_int(len(sc)),
                                _d(la), _d(cen))
    return la, cen


def boys0(T: float) -> float:
    return float(lib().orc_boys0(float(T)))


def aux_metric(log_alpha, centers, lam=0.0, omega=0.0):
    """gs_dft/coulomb/ri.py:63-76,267-275 (+ shift_diag); omega != 0: the erf(omega r)/r metric."""
    la, cen = _f64(log_alpha), _f64(centers)
    N = la.shape[0]
    V = np.empty((N, N))
    lib().orc_aux_metric(_i64(N), _d(la), _d(cen), ctypes.c_double(lam), ctypes.c_double(omega),
                         _d(V))
    return V


def aux_metric_rows(log_alpha, centers, rows, lam=0.0, omega=0.0):
    """Rows ``rows`` of aux_metric's V (len(rows), N), without forming the rest."""
    la, cen = _f64(log_alpha), _f64(centers)
    N = la.shape[0]
    r = np.ascontiguousarray(rows, dtype=np.int64)
    if r.size and (r.min() < 0 or r.max() >= N):
        raise IndexError("aux_metric_rows: row index out of range")
    V = np.empty((r.shape[0], N))
    lib().orc_aux_metric_rows(_i64(N), _d(la), _d(cen), ctypes.c_double(lam),
                              ctypes.c_double(omega), _i64(r.shape[0]),
                              r.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)), _d(V))
    return V


def cholesky(V):
    L = np.array(V, dtype=np.float64, copy=True, order="C")
    rc = lib().orc_cholesky(_i64(L.shape[0]), _d(L))
    if rc:
        raise np.linalg.LinAlgError("oracle Cholesky: matrix not positive definite")
    return L


def cho_solve(L, gamma):
    L, g = _f64(L), _f64(gamma)
    d = np.empty_like(g)
    lib().orc_cho_solve(_i64(L.shape[0]), _d(L), _d(g), _d(d))
    return d


def three_center_block(quat, log_scale, centers, log_alpha, aux_centers, pi, pj):
    quat, log_scale, centers = _f64(quat), _f64(log_scale), _f64(centers)
    la, ac, pi, pj = _f64(log_alpha), _f64(aux_centers), _i32(pi), _i32(pj)
    N, n = la.shape[0], pi.shape[0]
    B = np.empty((N, n))
    lib().orc_three_center_block(_i64(quat.shape[0]), _d(quat), _d(log_scale), _d(centers),
                                 _i64(N), _d(la), _d(ac), _i64(n), pi.ctypes.data_as(_I32),
                                 pj.ctypes.data_as(_I32), _d(B))
    return B


def gamma(quat, log_scale, centers, C, occ, log_alpha, aux_centers, pi, pj, weight):
    quat, log_scale, centers = _f64(quat), _f64(log_scale), _f64(centers)
    C, occ, la, ac = _f64(C), _f64(occ), _f64(log_alpha), _f64(aux_centers)
    pi, pj, w = _i32(pi), _i32(pj), _f64(weight)
    N = la.shape[0]
    g = np.empty(N)
    lib().orc_gamma(_i64(quat.shape[0]), _d(quat), _d(log_scale), _d(centers), _i64(C.shape[1]),
                    _d(C), _d(occ), _i64(N), _d(la), _d(ac), _i64(pi.shape[0]),
                    pi.ctypes.data_as(_I32), pj.ctypes.data_as(_I32), _d(w), _d(g))
    return g


def gamma_vjp(quat, log_scale, centers, C, occ, log_alpha, aux_centers, pi, pj, weight, dgamma):
    """(J, dquat, dlog_scale, dcenters, dC) for the upstream cotangent ``dgamma``."""
    quat, log_scale, centers = _f64(quat), _f64(log_scale), _f64(centers)
    C, occ, la, ac = _f64(C), _f64(occ), _f64(log_alpha), _f64(aux_centers)
    pi, pj, w, dg = _i32(pi), _i32(pj), _f64(weight), _f64(dgamma)
    M, k, n = quat.shape[0], C.shape[1], pi.shape[0]
    J = np.empty(n)
    dq = np.empty((M, 4))
    dl = np.empty((M, 3))
    dc = np.empty((M, 3))
    dC = np.empty((M, k))
    lib().orc_gamma_vjp(_i64(M), _d(quat), _d(log_scale), _d(centers), _i64(k), _d(C), _d(occ),
                        _i64(la.shape[0]), _d(la), _d(ac), _i64(n), pi.ctypes.data_as(_I32),
                        pj.ctypes.data_as(_I32), _d(w), _d(dg), _d(J), _d(dq), _d(dl), _d(dc),
                        _d(dC))
    return J, dq, dl, dc, dC


def dfj_energy(quat, log_scale, centers, C, occ, log_alpha, aux_centers, pi, pj, weight, lam):
    """(E_J, gamma, d, L) following gs_dft/coulomb/ri.py:485-494 with the refresh factor."""
    g = gamma(quat, log_scale, centers, C, occ, log_alpha, aux_centers, pi, pj, weight)
    L = cholesky(aux_metric(log_alpha, aux_centers, lam))
    d = cho_solve(L, g)
    return 0.5 * float(np.dot(g, d)), g, d, L


def dfj_grad(quat, log_scale, centers, C, occ, log_alpha, aux_centers, pi, pj, weight, lam):
    """(E_J, J, dquat, dlog_scale, dcenters, dC) of E_J = 1/2 gamma^T (V + lam I)^-1 gamma."""
    E, g, d, _L = dfj_energy(quat, log_scale, centers, C, occ, log_alpha, aux_centers, pi, pj,
                             weight, lam)
    return (E,) + gamma_vjp(quat, log_scale, centers, C, occ, log_alpha, aux_centers, pi, pj,
                            weight, d)


def nuclear_pairs(quat, log_scale, centers, pi, pj, atom_coords, atom_charges):
    """V (n) of gs_dft/screening/pairs.py:348-370 for the listed pairs."""
    quat, log_scale, centers = _f64(quat), _f64(log_scale), _f64(centers)
    pi, pj = _i32(pi), _i32(pj)
    R, Z = _f64(atom_coords).reshape(-1, 3), _f64(atom_charges).reshape(-1)
    V = np.empty(pi.shape[0])
    lib().orc_nuclear_pairs(_i64(quat.shape[0]), _d(quat), _d(log_scale), _d(centers),
                            _i64(pi.shape[0]), pi.ctypes.data_as(_I32), pj.ctypes.data_as(_I32),
                            _i64(R.shape[0]), _d(R), _d(Z), _d(V))
    return V


def external_energy(quat, log_scale, centers, C, occ, pi, pj, weight, atom_coords, atom_charges):
    """E_ext = sum_a w_a P_a V_a (gs_dft/screening/pairs.py:409-440)."""
    quat, log_scale, centers = _f64(quat), _f64(log_scale), _f64(centers)
    C, occ, pi, pj, w = _f64(C), _f64(occ), _i32(pi), _i32(pj), _f64(weight)
    R, Z = _f64(atom_coords).reshape(-1, 3), _f64(atom_charges).reshape(-1)
    return float(lib().orc_external_energy(
        _i64(quat.shape[0]), _d(quat), _d(log_scale), _d(centers), _i64(C.shape[1]), _d(C),
        _d(occ), _i64(pi.shape[0]), pi.ctypes.data_as(_I32), pj.ctypes.data_as(_I32), _d(w),
        _i64(R.shape[0]), _d(R), _d(Z)))


def eri_block(quat, log_scale, centers, ai, aj, bi, bj):
    """(a|b) (na, nb) of gs_dft/coulomb/stream.py:249-281."""
    quat, log_scale, centers = _f64(quat), _f64(log_scale), _f64(centers)
    ai, aj, bi, bj = _i32(ai), _i32(aj), _i32(bi), _i32(bj)
    out = np.empty((ai.shape[0], bi.shape[0]))
    lib().orc_eri_block(_i64(quat.shape[0]), _d(quat), _d(log_scale), _d(centers),
                        _i64(ai.shape[0]), ai.ctypes.data_as(_I32), aj.ctypes.data_as(_I32),
                        _i64(bi.shape[0]), bi.ctypes.data_as(_I32), bj.ctypes.data_as(_I32),
                        _d(out))
    return out


def exact_coulomb(quat, log_scale, centers, C, occ, pi, pj, weight):
    """(E_J, Jvec) of gs_dft/coulomb/stream.py:296-320 over the listed pairs."""
    quat, log_scale, centers = _f64(quat), _f64(log_scale), _f64(centers)
    C, occ, pi, pj, w = _f64(C), _f64(occ), _i32(pi), _i32(pj), _f64(weight)
    J = np.empty(pi.shape[0])
    E = lib().orc_exact_coulomb(_i64(quat.shape[0]), _d(quat), _d(log_scale), _d(centers),
                                _i64(C.shape[1]), _d(C), _d(occ), _i64(pi.shape[0]),
                                pi.ctypes.data_as(_I32), pj.ctypes.data_as(_I32), _d(w), _d(J))
    return float(E), J


def exchange_energy(quat, log_scale, centers, C, log_alpha, aux_centers, pi, pj, valid, lam,
                    omega=0.0):
    """Screened RI-K energy following gs_dft/coulomb/ri.py:497-544:
    D[P,o,o'] = sum over the valid listed pairs (i, k) of C_io C_ko' (P|ik) (``valid`` read as a
    mask, ri.py:529), M = sum_oo' D[P,o,o'] D[Q,o,o'] (ri.py:532), and
    E_K = -tr(solve(V + lam I, M)) with a dense solve (ri.py:544). omega != 0: the long-range
    exchange, (P|ik) with the rule lr_quad_table(omega) (ri.py:149,231-235) and V the erf metric
    (ri.py:543). Returns (E_K, D)."""
    C = _f64(C)
    pi_, pj_ = np.asarray(pi, dtype=np.int64), np.asarray(pj, dtype=np.int64)
    if omega:
        with node_rule(*lr_quad_table(omega)):
            B = three_center_block(quat, log_scale, centers, log_alpha, aux_centers, pi, pj)
    else:
        B = three_center_block(quat, log_scale, centers, log_alpha, aux_centers, pi, pj)
    m = (np.asarray(valid) != 0).astype(np.float64)
    D = np.einsum("Ap,po,pq->Aoq", B, C[pi_] * m[:, None], C[pj_], optimize=True)
    Mmat = np.einsum("Aoq,Boq->AB", D, D, optimize=True)
    V = aux_metric(log_alpha, aux_centers, lam, omega)
    return -float(np.trace(np.linalg.solve(V, Mmat))), D


def set_threads(n: int) -> None:
    os.environ["OMP_NUM_THREADS"] = str(int(n))
