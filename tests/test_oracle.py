"""Pins the CPU oracle (oracle/c/oracle.c) before it is trusted as the parity checker.

Every check below is independent of the oracle's own formulas: closed forms (isotropic overlap,
Gaussian Coulomb integrals, point-charge limits), invariants (normalisation, symmetry, rotation
equivariance), LAPACK, brute force, a literal eigh-based restatement of the reference kernel in
torch (oracle/torch_ref.py) with autograd for gradients, and finite differences. The reference
holds no golden vectors for this path (every DF-J test in gs-dft is relational), so these are
the pins.
"""
import math
import re

import numpy as np
import pytest
import torch
from scipy.special import erf

from conftest import ROOT, rel_max


def _t(x, grad=False):
    t = torch.as_tensor(np.asarray(x), dtype=torch.float64).clone()
    return t.requires_grad_(grad) if grad else t


def _idx(a):
    return torch.as_tensor(np.asarray(a, dtype=np.int64))


# ----------------------------------------------------------------------------- node table

def test_quad_table_newton_matches_numpy_leggauss(orc):
    t, w = orc.quad_table(20)
    tn, wn = orc.reference_quad_table(20)
    # the half-line map amplifies node round-off by 1/(1-s) ~ 300 at the last node
    assert rel_max(t, tn) < 1e-13 and np.max(np.abs(w - wn) / wn) < 1e-12


def test_library_table_is_numpy_leggauss_bit_exact(orc):
    src = (ROOT / "gs-dft_amd" / "csrc" / "common.h").read_text()
    blocks = re.findall(r"constexpr double [tw]\[kNodes\] = \{(.*?)\};", src, re.S)
    assert len(blocks) == 2
    vals = [np.array([float.fromhex(v.strip()) for v in b.split(",")]) for b in blocks]
    tn, wn = orc.reference_quad_table(20)
    assert np.array_equal(vals[0], tn) and np.array_equal(vals[1], wn)


def test_quad_table_integrates_the_coulomb_kernel(orc):
    """sum_t w_t exp(-t^2 r^2) ~ sqrt(pi)/(2 r): the half-line rule behind 1/r (the 20 nodes are
    accurate to ~1e-3 relative at r ~ 0.1-10, which is why parity is against the same rule)."""
    t, w = orc.reference_quad_table(20)
    for r in (0.3, 1.0, 3.0):
        approx = np.sum(w * np.exp(-(t * r) ** 2))
        assert abs(approx - math.sqrt(math.pi) / (2 * r)) < 2e-3 * math.sqrt(math.pi) / (2 * r)


# ----------------------------------------------------------------------------- chart

def test_chart_matches_literal_restatement_and_closed_forms(orc, tr, wl):
    s = wl.make_small(40, 3, seed=3)
    A, N = orc.chart(s.quat, s.log_scale)
    At = tr.splat_A(_t(s.quat), _t(s.log_scale)).numpy()
    assert np.max(np.abs(A - At)) < 1e-14 * np.max(np.abs(At))
    # det A = exp(sum l), N = (8 det A / pi^3)^(1/4): eigen-structure closed forms. The chart
    # divides q by |q| + 1e-12 (spectral.py:35), so R is orthogonal only to ~2e-12 and these hold
    # to ~1e-11.
    assert np.max(np.abs(np.linalg.det(A) / np.exp(s.log_scale.sum(1)) - 1)) < 1e-10
    assert np.max(np.abs(N - (8 * np.exp(s.log_scale.sum(1)) / math.pi ** 3) ** 0.25) / N) < 1e-15
    ev = np.sort(np.linalg.eigvalsh(A), axis=1)
    assert np.max(np.abs(ev / np.sort(np.exp(s.log_scale), axis=1) - 1)) < 1e-10


def test_chart_rotation_equivariance(orc, tr, wl):
    """q -> q_Q (x) q gives A -> Q A Q^T (gs-dft tests/unit/test_splat_chart.py:35)."""
    s = wl.make_small(12, 3, seed=4)
    qQ = np.array([0.3, -0.5, 0.7, 0.2]); qQ /= np.linalg.norm(qQ)
    Q = tr.quat_to_rotation(_t(qQ)).numpy()
    aw, ax, ay, az = qQ
    b = s.quat
    qrot = np.stack([aw * b[:, 0] - ax * b[:, 1] - ay * b[:, 2] - az * b[:, 3],
                     aw * b[:, 1] + ax * b[:, 0] + ay * b[:, 3] - az * b[:, 2],
                     aw * b[:, 2] - ax * b[:, 3] + ay * b[:, 0] + az * b[:, 1],
                     aw * b[:, 3] + ax * b[:, 2] - ay * b[:, 1] + az * b[:, 0]], axis=1)
    A, _ = orc.chart(s.quat, s.log_scale)
    Ar, _ = orc.chart(qrot, s.log_scale)
    # equivariance holds to the chart's own orthogonality (~1e-11, see the |q| + 1e-12 above)
    assert np.max(np.abs(Ar - np.einsum("ij,mjk,lk->mil", Q, A, Q))) < 1e-10 * np.max(np.abs(A))


# ----------------------------------------------------------------------------- overlap

def test_overlap_isotropic_closed_form(orc):
    rng = np.random.default_rng(5)
    M = 30
    alpha = np.exp(rng.uniform(-2, 2, M))
    quat = np.tile([1.0, 0, 0, 0], (M, 1))
    ls = np.repeat(np.log(alpha)[:, None], 3, 1)
    mu = rng.normal(0, 1.5, (M, 3))
    pi = np.repeat(np.arange(M), M); pj = np.tile(np.arange(M), M)
    S = orc.overlap_pairs(quat, ls, mu, pi, pj)
    ai, aj = alpha[pi], alpha[pj]
    d2 = np.sum((mu[pi] - mu[pj]) ** 2, 1)
    ref = (2 * np.sqrt(ai * aj) / (ai + aj)) ** 1.5 * np.exp(-ai * aj / (ai + aj) * d2)
    assert np.max(np.abs(S - ref) / ref) < 1e-13


def test_overlap_normalised_symmetric_and_literal(orc, tr, wl):
    s = wl.make_small(25, 3, seed=6)
    M = s.M
    pi = np.repeat(np.arange(M), M); pj = np.tile(np.arange(M), M)
    S = orc.overlap_pairs(s.quat, s.log_scale, s.centers, pi, pj).reshape(M, M)
    # unit-normalised splats (to the chart's ~1e-11 orthogonality, spectral.py:35), symmetric,
    # and bounded by Cauchy-Schwarz
    assert np.max(np.abs(np.diag(S) - 1.0)) < 1e-10
    assert np.max(np.abs(S - S.T)) < 1e-14 * np.max(S)
    assert np.all(S <= 1.0 + 1e-10)
    St = tr.full_overlap_pairs(_t(s.quat), _t(s.log_scale), _t(s.centers), _idx(pi), _idx(pj))
    assert np.max(np.abs(S.reshape(-1) - St.numpy()) / St.numpy()) < 1e-13


# ----------------------------------------------------------------------------- pair list

def _dense_S(tr, s):
    M = s.M
    pi = np.repeat(np.arange(M), M); pj = np.tile(np.arange(M), M)
    return np.abs(tr.full_overlap_pairs(_t(s.quat), _t(s.log_scale), _t(s.centers), _idx(pi),
                                        _idx(pj)).numpy()).reshape(M, M)


@pytest.mark.parametrize("unique", [False, True])
@pytest.mark.parametrize("eps", [1e-2, 1e-5, 1e-9])
def test_pairs_are_the_thresholded_set_lexsorted(orc, tr, wl, unique, eps):
    """gs-dft tests/unit/test_device_pairs.py:50 and test_pair_tricks.py:229."""
    s = wl.make_small(60, 3, n_atoms=5, spread=4.0, seed=8)
    S = _dense_S(tr, s)
    M = s.M
    want = [(i, j) for i in range(M) for j in range(M) if S[i, j] > eps and (j >= i or not unique)]
    # knife-edge audit: no pair within 1e-10 relative of eps, so the literal/oracle ulp-level
    # differences cannot flip membership
    assert not np.any(np.abs(S - eps) < 1e-10 * eps)
    pi, pj, w, n_sig = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, eps, None, unique)
    assert n_sig == len(want) == len(pi)
    assert list(zip(pi.tolist(), pj.tolist())) == want
    exp_w = [(1.0 if i == j else 2.0) if unique else 1.0 for i, j in want]
    assert np.array_equal(w, exp_w)
    assert orc.count_significant(s.quat, s.log_scale, s.centers, eps, unique) == len(want)


@pytest.mark.parametrize("seed,spread", [(8, 4.0), (9, 10.0), (10, 2.0)])
def test_spatial_candidate_rules_cover_the_significant_set(orc, wl, seed, spread):
    """gs_dft/screening/pairs.py:167-197: the spatial candidates must be a superset of the
    significant pairs. Brute force over every candidate: neither the reference's radius rule
    (|d| < 1.25 (rc_i + rc_j), rc = sqrt(-ln eps / lambda_min), grid.py:76-82) nor the tighter
    bound |d|^2 < -ln eps (1/lambda_min,i + 1/lambda_min,j) that the GPU spatial path uses misses a
    significant pair; the largest |d|^2 / bound over the significant pairs is below 1."""
    s = wl.make_small(120, 3, n_atoms=6, spread=spread, seed=seed)
    for eps in (1e-3, 1e-7, 1e-11):
        r = orc.spatial_audit(s.quat, s.log_scale, s.centers, eps, False)
        assert r["n_sig"] == orc.count_significant(s.quat, s.log_scale, s.centers, eps, False)
        assert r["n_miss_ref"] == 0 and r["n_miss_bound"] == 0 and r["max_ratio"] < 1.0
        assert r["n_sig"] <= r["n_cand_bound"] <= r["n_cand_ref"]


def test_unique_covers_ordered_with_weights(orc, wl):
    """gs-dft tests/unit/test_pair_tricks.py:44."""
    s = wl.make_small(48, 3, n_atoms=6, spread=3.0, seed=9)
    pi, pj, w, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, 1e-6, None, False)
    ui, uj, uw, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, 1e-6, None, True)
    assert np.all(uj >= ui) and set(np.unique(uw)) <= {1.0, 2.0}
    assert int(uw.sum()) == len(pi)
    ordered = set(zip(pi.tolist(), pj.tolist()))
    assert all((i, j) in ordered for i, j in zip(ui.tolist(), uj.tolist()))


def test_padding_tail_and_full_lists(orc, wl):
    """gs-dft tests/unit/test_device_pairs.py:62,91,146 and test_pair_tricks.py:57."""
    s = wl.make_small(24, 3, seed=10)
    M = s.M
    pi, pj, w, n = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, 1e-7, None, False)
    pad = len(pi) + 37
    qi, qj, qw, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, 1e-7, pad, False)
    assert len(qi) == pad and np.array_equal(qi[:len(pi)], pi) and np.all(qw[len(pi):] == 0)
    assert np.all(qi[len(pi):] == 0) and np.all(qj[len(pi):] == 0)
    big = M * M + 500
    bi, _, bw, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, 1e-7, big, False)
    assert len(bi) == big
    for pad_to in (None, M * M, M * M + 313):
        fi, fj, fw, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, -1.0, pad_to, False)
        assert np.array_equal(fi[:M * M], np.repeat(np.arange(M), M))
        assert np.array_equal(fj[:M * M], np.tile(np.arange(M), M))
        assert np.all(fw[:M * M] == 1) and np.all(fw[M * M:] == 0)
    ui, uj, uw, _ = orc.neighbor_pairs(s.quat[:7], s.log_scale[:7], s.centers[:7], -1.0, None, True)
    assert len(ui) == 28 and uw.sum() == 49.0


def test_overflow_keeps_the_largest_exactly(orc, tr, wl):
    """gs-dft tests/unit/test_pair_tricks.py:260: the pad_to largest |S|, re-lexsorted, and
    ValueError beyond twice the pad (pairs.py:157-161)."""
    s = wl.make_small(40, 3, n_atoms=4, spread=3.0, seed=11)
    S = _dense_S(tr, s)
    M = s.M
    for unique in (False, True):
        mask = S > 1e-6
        if unique:
            mask &= np.triu(np.ones((M, M), bool))
        flat = np.nonzero(mask.reshape(-1))[0]
        vals = S.reshape(-1)[flat]
        pad = len(flat) // 2 + 1
        want = np.sort(flat[np.argsort(-vals, kind="stable")[:pad]])
        pi, pj, w, n_sig = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, 1e-6, pad, unique)
        got = pi.astype(np.int64) * M + pj
        assert n_sig == len(flat) and np.array_equal(got, want) and np.all(w > 0)
        with pytest.raises(ValueError):
            orc.neighbor_pairs(s.quat, s.log_scale, s.centers, 1e-6, len(flat) // 3, unique)


# ----------------------------------------------------------------------------- aux + metric

def test_product_aux_closed_form_and_literal(orc, tr, wl):
    s = wl.make_small(30, 3, seed=12)
    la, ac = orc.product_aux(s.quat, s.log_scale, s.centers, (0.5, 1.0, 2.0))
    lat, act = tr.init_product_aux(_t(s.quat), _t(s.log_scale), _t(s.centers), (0.5, 1.0, 2.0))
    assert np.max(np.abs(la - lat.numpy())) < 1e-14 and np.max(np.abs(ac - act.numpy())) < 1e-13
    # self-product exponent det(2A)^(1/3) = 2 exp(mean l) (to the chart's ~1e-11 orthogonality),
    # centre = the splat centre
    base = np.log(2.0) + s.log_scale.mean(1)
    M = s.M
    for k, sc in enumerate((0.5, 1.0, 2.0)):
        assert np.max(np.abs(la[k * M:(k + 1) * M] - (base + np.log(sc)))) < 1e-10
        assert np.max(np.abs(ac[k * M:(k + 1) * M] - s.centers)) < 1e-12
    assert len(la) == 3 * M                       # N_aux = mult * M (test_aux_mult.py:29)


def test_product_aux_of_listed_pairs(orc, wl):
    """Off-diagonal product aux (gs_dft/basis/isotropic.py:106-116): on the self-pairs it is the
    diagonal aux; for isotropic splats A = a I the product exponent det(A_i + A_j)^(1/3) is
    a_i + a_j at the centre (a_i mu_i + a_j mu_j) / (a_i + a_j); for anisotropic splats the
    exponent is numpy's det of the summed chart precisions; entries with valid 0 take
    alpha_0 = 1 (exponent = the scale) at their pair's product centre."""
    s = wl.make_small(30, 3, seed=12)
    M = s.M
    scales = (0.5, 1.0, 2.0)
    idx = np.arange(M)
    la, ac = orc.product_aux_pairs(s.quat, s.log_scale, s.centers, idx, idx, None, scales)
    ld, acd = orc.product_aux(s.quat, s.log_scale, s.centers, scales)
    assert np.array_equal(la, ld) and np.array_equal(ac, acd)
    rng = np.random.default_rng(3)
    a = np.exp(rng.uniform(-1, 1, M))
    quat = np.tile([1.0, 0, 0, 0], (M, 1))
    ls = np.repeat(np.log(a)[:, None], 3, 1)
    pi = rng.integers(0, M, 50).astype(np.int32)
    pj = rng.integers(0, M, 50).astype(np.int32)
    valid = (rng.uniform(size=50) > 0.2).astype(float) * 2.0
    la, ac = orc.product_aux_pairs(quat, ls, s.centers, pi, pj, valid, scales)
    n = len(pi)
    want_c = (a[pi, None] * s.centers[pi] + a[pj, None] * s.centers[pj]) / (a[pi] + a[pj])[:, None]
    for k, sc in enumerate(scales):
        blk = slice(k * n, (k + 1) * n)
        want = np.where(valid != 0, np.log((a[pi] + a[pj]) * sc), np.log(sc))
        assert np.max(np.abs(la[blk] - want)) < 1e-14
        assert np.max(np.abs(ac[blk] - want_c)) < 1e-13
    A, _ = orc.chart(s.quat, s.log_scale)
    la, _ = orc.product_aux_pairs(s.quat, s.log_scale, s.centers, pi, pj, None, (1.0,))
    assert np.max(np.abs(la - np.log(np.linalg.det(A[pi] + A[pj])) / 3.0)) < 1e-13


def _gauss_coulomb(a, A, b, B):
    """(s_a|1/r|s_b) of unit-L2-normalised s-Gaussians, textbook erf form."""
    NA, NB = (2 * a / math.pi) ** 0.75, (2 * b / math.pi) ** 0.75
    p = a * b / (a + b)
    R = np.linalg.norm(np.asarray(A) - np.asarray(B))
    pref = NA * NB * (math.pi / a) ** 1.5 * (math.pi / b) ** 1.5
    return pref * (erf(math.sqrt(p) * R) / R if R > 0 else 2 * math.sqrt(p / math.pi))


def test_metric_textbook_closed_form_and_limits(orc):
    rng = np.random.default_rng(13)
    N = 40
    la = rng.uniform(-2.5, 2.0, N)
    cen = rng.normal(0, 2.0, (N, 3))
    cen[5] = cen[4]                                        # a coincident pair (T = 0)
    V = orc.aux_metric(la, cen)
    beta = np.exp(la)
    ref = np.array([[_gauss_coulomb(beta[p], cen[p], beta[q], cen[q]) for q in range(N)]
                    for p in range(N)])
    assert np.max(np.abs(V - ref) / np.abs(ref)) < 1e-13
    assert np.max(np.abs(np.diag(V) - 4 * math.pi / beta) * beta) < 1e-13
    assert np.array_equal(V, V.T)
    # point-charge limit: charges (2 pi / beta)^(3/4) at large separation
    far = orc.aux_metric(np.log([0.8, 1.3]), np.array([[0, 0, 0], [0, 0, 60.0]]))
    q = (2 * math.pi / np.array([0.8, 1.3])) ** 0.75
    assert abs(far[0, 1] - q[0] * q[1] / 60.0) < 1e-12 * far[0, 1]
    assert abs(orc.boys0(0.0) - 1.0) < 1e-16 and abs(orc.boys0(1e-13) - (1 - 1e-13 / 3)) < 1e-16


@pytest.mark.parametrize("lam,omega", [(0.0, 0.0), (1e-8, 0.0), (1e-2, 0.7)])
def test_metric_rows_are_the_metric_rows(orc, lam, omega):
    """aux_metric_rows (the full-size tests' sampled rows) gives exactly the rows of aux_metric,
    the shift on the diagonal included; an out-of-range row is refused."""
    rng = np.random.default_rng(15)
    N = 57
    la = rng.uniform(-2.5, 2.0, N)
    cen = rng.normal(0, 2.0, (N, 3))
    V = orc.aux_metric(la, cen, lam, omega)
    rows = np.array([0, 3, 3, 56, 20])
    assert np.array_equal(orc.aux_metric_rows(la, cen, rows, lam, omega), V[rows])
    with pytest.raises(IndexError):
        orc.aux_metric_rows(la, cen, [N], lam, omega)


def test_cholesky_and_solve_match_lapack(orc, wl):
    s = wl.make_small(40, 3, seed=14)
    la, ac = orc.product_aux(s.quat, s.log_scale, s.centers, (0.5, 1.0, 2.0, 4.0))
    V = orc.aux_metric(la, ac, 1e-8)
    L = orc.cholesky(V)
    Ln = np.linalg.cholesky(V)
    assert np.max(np.abs(L - Ln)) < 1e-9 * np.max(np.abs(Ln))
    assert np.all(np.triu(L, 1) == 0)
    g = np.random.default_rng(0).normal(size=V.shape[0])
    d = orc.cho_solve(L, g)
    dn = np.linalg.solve(V, g)
    # relational bound of gs-dft tests/unit/test_refresh_cholv.py:24 (cho_solve == dense solve)
    assert abs(0.5 * g @ d - 0.5 * g @ dn) < 1e-10 * max(1.0, abs(0.5 * g @ dn))


# ----------------------------------------------------------------------------- three-centre

def test_three_centre_matches_literal_eigh_kernel(orc, tr, wl):
    s = wl.make_small(20, 3, seed=15)
    la, ac = orc.product_aux(s.quat, s.log_scale, s.centers, (0.5, 2.0))
    pi, pj, w, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, 1e-9, None, True)
    B = orc.three_center_block(s.quat, s.log_scale, s.centers, la, ac, pi, pj)
    A, N = tr.splat_A(_t(s.quat), _t(s.log_scale)), tr.splat_norm(_t(s.log_scale))
    Bt = tr.full_isobra_block(*tr.aux_quantities(_t(la), _t(ac)),
                              *tr.full_pair_quantities(A, _t(s.centers), N, _idx(pi), _idx(pj))).numpy()
    assert np.max(np.abs(B - Bt) / np.abs(Bt)) < 1e-12


def test_three_centre_structure_converges_to_boys(orc, tr):
    """Isotropic pair products: the (iso aux | pair) integral is the textbook s-s Coulomb
    integral. The reference's integrand (literal eigh form) under a 400-node rule reproduces the
    closed form to 1e-9, and the 20-node oracle agrees with the 20-node literal kernel; so the
    prefactor and node algebra are pinned independently of the 20-node table."""
    rng = np.random.default_rng(16)
    M = 6
    alpha = np.exp(rng.uniform(-1.5, 1.0, M))
    quat = np.tile([1.0, 0, 0, 0], (M, 1))
    ls = np.repeat(np.log(alpha)[:, None], 3, 1)
    mu = rng.normal(0, 1.2, (M, 3))
    pi = np.repeat(np.arange(M), M); pj = np.tile(np.arange(M), M)
    la = rng.uniform(-1.0, 1.5, 5)
    ac = rng.normal(0, 1.5, (5, 3))
    x, wl_ = np.polynomial.legendre.leggauss(400)
    sgl = (x + 1) / 2
    table = ([float(v) for v in sgl / (1 - sgl)], [float(v) for v in (wl_ / 2) / (1 - sgl) ** 2])
    A, N = tr.splat_A(_t(quat), _t(ls)), tr.splat_norm(_t(ls))
    Ah, P, KN = tr.full_pair_quantities(A, _t(mu), N, _idx(pi), _idx(pj))
    Bconv = tr.full_isobra_block(*tr.aux_quantities(_t(la), _t(ac)), Ah, P, KN, table).numpy()
    beta = np.exp(la)
    p = alpha[pi] + alpha[pj]
    for a_ in range(len(pi)):
        for P_ in range(len(la)):
            # pair product = KN_a * exp(-p |r - P|^2); aux = KN_P exp(-beta |r - R|^2)
            R = np.linalg.norm(ac[P_] - P.numpy()[a_])
            red = beta[P_] * p[a_] / (beta[P_] + p[a_])
            F0 = erf(math.sqrt(red) * R) / (R * math.sqrt(red)) * math.sqrt(math.pi) / 2 if R > 0 else 1.0
            ref = ((2 * beta[P_] / math.pi) ** 0.75 * KN.numpy()[a_] * 2 * math.pi ** 2.5
                   / (beta[P_] * p[a_] * math.sqrt(beta[P_] + p[a_])) * F0)
            assert abs(Bconv[P_, a_] - ref) < 1e-9 * abs(ref)
    B20 = orc.three_center_block(quat, ls, mu, la, ac, pi, pj)
    B20t = tr.full_isobra_block(*tr.aux_quantities(_t(la), _t(ac)), Ah, P, KN).numpy()
    assert np.max(np.abs(B20 - B20t) / np.abs(B20t)) < 1e-12


# ----------------------------------------------------------------------------- gamma / E_J / grads

def _system(wl, orc, M=24, k=5, seed=1, n_scales=2, eps=1e-7, unique=True):
    s = wl.make_small(M, k, n_atoms=3, seed=seed, n_scales=n_scales)
    la, ac = orc.product_aux(s.quat, s.log_scale, s.centers, s.scales)
    pi, pj, w, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, eps, None, unique)
    return s, la, ac, pi, pj, w


def test_gamma_matches_literal(orc, tr, wl):
    s, la, ac, pi, pj, w = _system(wl, orc)
    g = orc.gamma(s.quat, s.log_scale, s.centers, s.C, s.occ, la, ac, pi, pj, w)
    gt = tr.gamma_screened(_t(s.quat), _t(s.log_scale), _t(s.centers), _t(s.C), _t(s.occ),
                           _t(la), _t(ac), _idx(pi), _idx(pj), _t(w), chunk=50)
    assert rel_max(g, gt.numpy()) < 1e-13


def test_unique_equals_ordered_values_and_gradients(orc, wl):
    """gs-dft tests/unit/test_pair_tricks.py:81 (relational: the unique list with weights 2 - d_ij
    must reproduce the ordered list)."""
    s, la, ac, ui, uj, uw = _system(wl, orc, unique=True)
    _, _, _, oi, oj, ow = _system(wl, orc, unique=False)
    gu = orc.gamma(s.quat, s.log_scale, s.centers, s.C, s.occ, la, ac, ui, uj, uw)
    go = orc.gamma(s.quat, s.log_scale, s.centers, s.C, s.occ, la, ac, oi, oj, ow)
    assert rel_max(gu, go) < 1e-12
    gu_ = orc.gamma_vjp(s.quat, s.log_scale, s.centers, s.C, s.occ, la, ac, ui, uj, uw, gu)
    go_ = orc.gamma_vjp(s.quat, s.log_scale, s.centers, s.C, s.occ, la, ac, oi, oj, ow, go)
    for a, b in zip(gu_[1:], go_[1:]):
        assert rel_max(a, b) < 1e-11


def test_energy_and_gradients_match_autograd_of_literal(orc, tr, wl):
    s, la, ac, pi, pj, w = _system(wl, orc, M=20, k=4, seed=2)
    lam = 1e-8
    E, J, dq, dl, dc, dC = orc.dfj_grad(s.quat, s.log_scale, s.centers, s.C, s.occ, la, ac,
                                        pi, pj, w, lam)
    q, l, c, C = (_t(a, True) for a in (s.quat, s.log_scale, s.centers, s.C))
    g = tr.gamma_screened(q, l, c, C, _t(s.occ), _t(la), _t(ac), _idx(pi), _idx(pj), _t(w))
    V = tr.aux_metric(_t(la), _t(ac)) + lam * torch.eye(len(la), dtype=torch.float64)
    Et = tr.coulomb_solve(g, torch.linalg.cholesky(V))
    Et.backward()
    assert abs(E - Et.item()) < 1e-11 * abs(E) and E > 0
    for a, b in ((dq, q.grad), (dl, l.grad), (dc, c.grad), (dC, C.grad)):
        assert rel_max(a, b.numpy()) < 1e-9
    # J_a = dE/dq_a: the derivative of the literal E w.r.t. the pair densities
    gq = torch.zeros(len(pi), dtype=torch.float64, requires_grad=True)
    qa = _t(w) * torch.sum(_t(s.occ)[None] * _t(s.C)[_idx(pi)] * _t(s.C)[_idx(pj)], 1)
    A, N = tr.splat_A(_t(s.quat), _t(s.log_scale)), tr.splat_norm(_t(s.log_scale))
    B = tr.full_isobra_block(*tr.aux_quantities(_t(la), _t(ac)),
                             *tr.full_pair_quantities(A, _t(s.centers), N, _idx(pi), _idx(pj)))
    Eq = tr.coulomb_solve(B @ (qa + gq), torch.linalg.cholesky(V))
    Eq.backward()
    assert rel_max(J, gq.grad.numpy()) < 1e-10


def test_gradients_finite_differences(orc, wl):
    """Central differences of the oracle's own E_J (coarse: 1e-6) on a few coordinates."""
    s, la, ac, pi, pj, w = _system(wl, orc, M=16, k=3, seed=3)
    lam = 1e-8

    def energy(quat, ls, cen, C):
        return orc.dfj_energy(quat, ls, cen, C, s.occ, la, ac, pi, pj, w, lam)[0]

    E, J, dq, dl, dc, dC = orc.dfj_grad(s.quat, s.log_scale, s.centers, s.C, s.occ, la, ac,
                                        pi, pj, w, lam)
    h = 1e-5
    for which, grad in ((0, dq), (1, dl), (2, dc), (3, dC)):
        base = [s.quat.copy(), s.log_scale.copy(), s.centers.copy(), s.C.copy()]
        for (r, col) in ((0, 0), (3, 1), (7, grad.shape[1] - 1)):
            up = [b.copy() for b in base]; dn = [b.copy() for b in base]
            up[which][r, col] += h; dn[which][r, col] -= h
            fd = (energy(*up) - energy(*dn)) / (2 * h)
            assert abs(fd - grad[r, col]) < 1e-6 * max(1.0, np.max(np.abs(grad)))


def test_gradients_finite_at_isotropic_splats(orc, wl):
    """The reference's eigh VJP is NaN at exactly degenerate Ah (gs_dft/coulomb/ri.py:139-143);
    the invariant form is smooth there, and its gradient matches finite differences."""
    s = wl.make_small(10, 3, seed=4)
    ls = np.repeat(s.log_scale[:, :1], 3, 1)                   # isotropic splats
    la, ac = orc.product_aux(s.quat, ls, s.centers, (1.0,))
    pi, pj, w, _ = orc.neighbor_pairs(s.quat, ls, s.centers, 1e-7, None, True)
    E, J, dq, dl, dc, dC = orc.dfj_grad(s.quat, ls, s.centers, s.C, s.occ, la, ac, pi, pj, w, 1e-8)
    for a in (dq, dl, dc, dC):
        assert np.all(np.isfinite(a))
    assert np.max(np.abs(dq)) < 1e-8 * max(1.0, np.max(np.abs(dc)))   # dA/dq = 0 at isotropy
    h = 1e-5
    c2 = s.centers.copy(); c2[2, 1] += h
    c3 = s.centers.copy(); c3[2, 1] -= h
    fd = (orc.dfj_energy(s.quat, ls, c2, s.C, s.occ, la, ac, pi, pj, w, 1e-8)[0]
          - orc.dfj_energy(s.quat, ls, c3, s.C, s.occ, la, ac, pi, pj, w, 1e-8)[0]) / (2 * h)
    assert abs(fd - dc[2, 1]) < 1e-6 * max(1.0, abs(dc[2, 1]))


def test_full_list_equals_dense_sum(orc, wl):
    """Screened gamma over the full ordered list == the dense contraction over all M^2 pairs
    with P = C C^T (gs-dft tests/unit/test_coulomb_df.py:107)."""
    s = wl.make_small(12, 3, seed=5)
    la, ac = orc.product_aux(s.quat, s.log_scale, s.centers, (1.0,))
    pi, pj, w, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, -1.0, None, False)
    g = orc.gamma(s.quat, s.log_scale, s.centers, s.C, s.occ, la, ac, pi, pj, w)
    B = orc.three_center_block(s.quat, s.log_scale, s.centers, la, ac, pi, pj)
    P = s.C @ np.diag(s.occ) @ s.C.T
    assert rel_max(g, B @ P.reshape(-1)) < 1e-13


# ----------------------------------------------------------------------------- nuclear attraction

def _nuc_system(wl, orc, M=24, k=5, seed=3, unique=True):
    s = wl.make_small(M, k, n_atoms=3, seed=seed)
    pi, pj, w, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, 1e-7, None, unique)
    return s, pi, pj, w


def test_nuclear_pairs_match_literal_restatement(orc, tr, wl):
    """gs_dft/screening/pairs.py:348-370: the C oracle against the torch line-by-line form."""
    for seed in (3, 4):
        s, pi, pj, w = _nuc_system(wl, orc, seed=seed)
        V = orc.nuclear_pairs(s.quat, s.log_scale, s.centers, pi, pj, s.atoms, s.charges)
        Vt = tr.full_nuclear_pairs(_t(s.quat), _t(s.log_scale), _t(s.centers), _idx(pi),
                                   _idx(pj), _t(s.atoms), _t(s.charges)).numpy()
        assert np.all(V < 0) and np.max(np.abs(V - Vt) / np.abs(Vt)) < 1e-13
        E = orc.external_energy(s.quat, s.log_scale, s.centers, s.C, s.occ, pi, pj, w, s.atoms,
                                s.charges)
        Et = tr.screened_external_energy(_t(s.quat), _t(s.log_scale), _t(s.centers), _t(s.C),
                                         _t(s.occ), _idx(pi), _idx(pj), _t(w), _t(s.atoms),
                                         _t(s.charges)).item()
        assert abs(E - Et) < 1e-13 * abs(Et)


def test_nuclear_invariant_form_equals_literal_node():
    """The library evaluates det(A + sI) and the exponent through the invariants I1, I2, I3 and
    q0 = |d|^2, q1 = d.A d, q2 = |A d|^2: det = Pn(s) = I3 + s (I2 + s (I1 + s)) and
    t^2 |d|^2 - t^4 d.adj(B) d / det B = s Qn(s) / Pn(s), Qn = I3 q0 + s (I1 q1 - q2) + s^2 q1,
    with s = t^2 (Cayley-Hamilton)."""
    rng = np.random.default_rng(5)
    for _ in range(200):
        X = rng.normal(size=(3, 3))
        A = X @ X.T + rng.uniform(0.05, 3.0) * np.eye(3)
        d = rng.normal(0, 3.0, 3)
        t = rng.uniform(0.01, 30.0)
        s = t * t
        B = A + s * np.eye(3)
        adjB = np.linalg.inv(B) * np.linalg.det(B)
        expo = s * (d @ d) - s * s * (d @ adjB @ d) / np.linalg.det(B)
        I1, I3 = np.trace(A), np.linalg.det(A)
        I2 = 0.5 * (I1 * I1 - np.trace(A @ A))
        Pn = I3 + s * (I2 + s * (I1 + s))
        q0, q1, q2 = d @ d, d @ A @ d, (A @ d) @ (A @ d)
        Qn = I3 * q0 + s * ((I1 * q1 - q2) + s * q1)
        assert abs(Pn - np.linalg.det(B)) < 1e-11 * abs(Pn)
        assert abs(s * Qn / Pn - expo) < 1e-10 * max(abs(expo), 1.0)


def test_nuclear_converges_to_point_charge_closed_form(orc, tr):
    """Isotropic pair products p = a_i + a_j: the electron-nucleus integral of
    exp(-p |r - P|^2) with a charge Z at R is -Z (2 pi / p) F0(p |P - R|^2). The reference's node
    formula under a 400-node rule reproduces it to 1e-10, and the 20-node oracle agrees with the
    20-node literal form, so prefactor and node algebra are pinned apart from the table."""
    rng = np.random.default_rng(21)
    M = 5
    alpha = np.exp(rng.uniform(-1.5, 1.0, M))
    quat = rng.normal(size=(M, 4))
    ls = np.repeat(np.log(alpha)[:, None], 3, 1)
    mu = rng.normal(0, 1.2, (M, 3))
    pi = np.repeat(np.arange(M), M); pj = np.tile(np.arange(M), M)
    atoms = rng.normal(0, 2.0, (4, 3)); Z = np.array([1.0, 6.0, 8.0, 7.0])
    x, wl_ = np.polynomial.legendre.leggauss(400)
    sgl = (x + 1) / 2
    table = ([float(v) for v in sgl / (1 - sgl)], [float(v) for v in (wl_ / 2) / (1 - sgl) ** 2])
    Vc = tr.full_nuclear_pairs(_t(quat), _t(ls), _t(mu), _idx(pi), _idx(pj), _t(atoms), _t(Z),
                               table).numpy()
    A, N = tr.splat_A(_t(quat), _t(ls)), tr.splat_norm(_t(ls))
    _, P, KN = tr.full_pair_quantities(A, _t(mu), N, _idx(pi), _idx(pj))
    P, KN = P.numpy(), KN.numpy()
    p = alpha[pi] + alpha[pj]
    for a_ in range(len(pi)):
        ref = 0.0
        for at in range(len(Z)):
            T = p[a_] * np.sum((P[a_] - atoms[at]) ** 2)
            F0 = 0.5 * math.sqrt(math.pi / T) * erf(math.sqrt(T)) if T > 1e-12 else 1.0 - T / 3
            ref -= Z[at] * 2 * math.pi / p[a_] * F0
        assert abs(Vc[a_] - KN[a_] * ref) < 1e-10 * abs(KN[a_] * ref)
    V20 = orc.nuclear_pairs(quat, ls, mu, pi, pj, atoms, Z)
    V20t = tr.full_nuclear_pairs(_t(quat), _t(ls), _t(mu), _idx(pi), _idx(pj), _t(atoms),
                                 _t(Z)).numpy()
    assert np.max(np.abs(V20 - V20t) / np.abs(V20t)) < 1e-13


def test_external_energy_invariances(orc, wl):
    """Moving splats and nuclei together (translation, rotation) leaves E_ext unchanged, the
    unique list with weights 2 - delta_ij equals the ordered list, and padding adds nothing."""
    s, pi, pj, w = _nuc_system(wl, orc)
    E = orc.external_energy(s.quat, s.log_scale, s.centers, s.C, s.occ, pi, pj, w, s.atoms,
                            s.charges)
    shift = np.array([1.3, -0.7, 2.1])
    Es = orc.external_energy(s.quat, s.log_scale, s.centers + shift, s.C, s.occ, pi, pj, w,
                             s.atoms + shift, s.charges)
    assert abs(Es - E) < 1e-12 * abs(E)
    th = 0.7
    Rz = np.array([[math.cos(th), -math.sin(th), 0], [math.sin(th), math.cos(th), 0], [0, 0, 1]])
    qz = np.array([math.cos(th / 2), 0, 0, math.sin(th / 2)])     # rotation about z by th
    w0, x0, y0, z0 = qz
    qr = np.array([[w0 * a - x0 * b - y0 * c - z0 * d, w0 * b + x0 * a + y0 * d - z0 * c,
                    w0 * c - x0 * d + y0 * a + z0 * b, w0 * d + x0 * c - y0 * b + z0 * a]
                   for a, b, c, d in s.quat])
    Er = orc.external_energy(qr, s.log_scale, s.centers @ Rz.T, s.C, s.occ, pi, pj, w,
                             s.atoms @ Rz.T, s.charges)
    assert abs(Er - E) < 1e-11 * abs(E)
    po, qo, wo, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, 1e-7, None, False)
    Eo = orc.external_energy(s.quat, s.log_scale, s.centers, s.C, s.occ, po, qo, wo, s.atoms,
                             s.charges)
    assert abs(Eo - E) < 1e-12 * abs(E)
    pad = len(pi) + 17
    pp, qp, wp, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, 1e-7, pad, True)
    Ep = orc.external_energy(s.quat, s.log_scale, s.centers, s.C, s.occ, pp, qp, wp, s.atoms,
                             s.charges)
    assert Ep == E


def test_external_energy_autograd_matches_finite_differences(orc, tr, wl):
    """Autograd of the literal restatement (the gradient reference for the GPU) against central
    differences of the C oracle, for nuclear coordinates and splat leaves."""
    s, pi, pj, w = _nuc_system(wl, orc, M=16, seed=7)
    args = [_t(s.quat, True), _t(s.log_scale, True), _t(s.centers, True), _t(s.C, True)]
    R = _t(s.atoms, True)
    E = tr.screened_external_energy(*args, _t(s.occ), _idx(pi), _idx(pj), _t(w), R,
                                    _t(s.charges))
    E.backward()
    h = 1e-5

    def f(**kw):
        v = dict(quat=s.quat, log_scale=s.log_scale, centers=s.centers, C=s.C, atoms=s.atoms)
        v.update(kw)
        return orc.external_energy(v["quat"], v["log_scale"], v["centers"], v["C"], s.occ, pi, pj,
                                   w, v["atoms"], s.charges)

    for name, arr, g in (("atoms", s.atoms, R.grad), ("centers", s.centers, args[2].grad),
                         ("log_scale", s.log_scale, args[1].grad), ("quat", s.quat, args[0].grad)):
        for idx in [(0, 0), (1, 2), (arr.shape[0] - 1, 1)]:
            up, dn = arr.copy(), arr.copy()
            up[idx] += h; dn[idx] -= h
            fd = (f(**{name: up}) - f(**{name: dn})) / (2 * h)
            assert abs(fd - g[idx].item()) < 1e-6 * max(1.0, abs(fd)), (name, idx)


# ----------------------------------------------------------------------------- exact pair-pair Coulomb

def test_eri_matches_literal_schur_and_is_symmetric(orc, tr, wl):
    """gs_dft/coulomb/stream.py:249-281: the C oracle against the torch line-by-line Schur form,
    and (a|b) = (b|a)."""
    s, pi, pj, w = _nuc_system(wl, orc, seed=3)
    B = orc.eri_block(s.quat, s.log_scale, s.centers, pi, pj, pi, pj)
    Bt = tr.full_eri_block_schur(_t(s.quat), _t(s.log_scale), _t(s.centers), _idx(pi), _idx(pj),
                                 _idx(pi), _idx(pj)).numpy()
    assert np.max(np.abs(B - Bt) / np.abs(Bt)) < 1e-12
    assert np.max(np.abs(B - B.T)) < 1e-13 * np.max(np.abs(B))
    E, J = orc.exact_coulomb(s.quat, s.log_scale, s.centers, s.C, s.occ, pi, pj, w)
    Et = tr.screened_coulomb_energy(_t(s.quat), _t(s.log_scale), _t(s.centers), _t(s.C),
                                    _t(s.occ), _idx(pi), _idx(pj), _t(w)).item()
    assert abs(E - Et) < 1e-13 * abs(Et)


def test_eri_division_free_form_equals_schur_form(orc, wl):
    """The library evaluates each node as det(I + sT)^(-1/2) exp(-s d.(I + sT)^-1 d) with
    T = A_a^-1 + A_b^-1 and d = P_a - P_b, through J1..J3 = invariants of T and
    p0 = |d|^2, p1 = J1 p0 - d.T d, p2 = d.adj(T) d (Cayley-Hamilton); the prefactor
    2 pi^2.5 KN_a KN_b (det A_a det A_b)^(-1/2). Checked against the reference's Schur form."""
    s, pi, pj, w = _nuc_system(wl, orc, seed=4)
    B = orc.eri_block(s.quat, s.log_scale, s.centers, pi, pj, pi, pj)
    A9, N = orc.chart(s.quat, s.log_scale)
    Ah, P, KN = orc.pair_quantities(A9, s.centers, N, pi, pj)
    tq, wq = orc.reference_quad_table(20)
    rng = np.random.default_rng(0)
    for a, b in rng.integers(0, len(pi), (300, 2)):
        T = np.linalg.inv(Ah[a]) + np.linalg.inv(Ah[b])
        d = P[a] - P[b]
        J1, J3 = np.trace(T), np.linalg.det(T)
        J2 = 0.5 * (J1 * J1 - np.trace(T @ T))
        p0 = d @ d
        p1 = J1 * p0 - d @ T @ d
        p2 = d @ (np.linalg.inv(T) * J3) @ d
        sv = tq * tq
        E = 1 + sv * (J1 + sv * (J2 + sv * J3))
        F = np.sum(wq * E ** -0.5 * np.exp(-sv * (p0 + sv * (p1 + sv * p2)) / E))
        val = (KN[a] * KN[b] * 2 * math.pi ** 2.5
               * (np.linalg.det(Ah[a]) * np.linalg.det(Ah[b])) ** -0.5 * F)
        assert abs(val - B[a, b]) < 1e-12 * abs(B[a, b])


def test_eri_converges_to_isotropic_closed_form(tr):
    """Isotropic pair products p, q: (a|b) = KN_a KN_b 2 pi^2.5 / (p q sqrt(p + q)) F0(rho R^2),
    rho = p q / (p + q) -- the reference's node formula under a 400-node rule reproduces it."""
    rng = np.random.default_rng(31)
    M = 5
    alpha = np.exp(rng.uniform(-1.0, 1.0, M))
    quat = rng.normal(size=(M, 4))
    ls = np.repeat(np.log(alpha)[:, None], 3, 1)
    mu = rng.normal(0, 1.5, (M, 3))
    pi = np.repeat(np.arange(M), M); pj = np.tile(np.arange(M), M)
    x, wl_ = np.polynomial.legendre.leggauss(400)
    sgl = (x + 1) / 2
    table = ([float(v) for v in sgl / (1 - sgl)], [float(v) for v in (wl_ / 2) / (1 - sgl) ** 2])
    Bc = tr.full_eri_block_schur(_t(quat), _t(ls), _t(mu), _idx(pi), _idx(pj), _idx(pi),
                                 _idx(pj), table).numpy()
    A, N = tr.splat_A(_t(quat), _t(ls)), tr.splat_norm(_t(ls))
    _, P, KN = tr.full_pair_quantities(A, _t(mu), N, _idx(pi), _idx(pj))
    P, KN = P.numpy(), KN.numpy()
    pp = alpha[pi] + alpha[pj]
    for a in range(len(pi)):
        for b in range(len(pi)):
            rho = pp[a] * pp[b] / (pp[a] + pp[b])
            T = rho * np.sum((P[a] - P[b]) ** 2)
            F0 = 0.5 * math.sqrt(math.pi / T) * erf(math.sqrt(T)) if T > 1e-12 else 1.0 - T / 3
            ref = KN[a] * KN[b] * 2 * math.pi ** 2.5 / (pp[a] * pp[b] * math.sqrt(pp[a] + pp[b])) * F0
            assert abs(Bc[a, b] - ref) < 1e-10 * abs(ref)


def test_exact_coulomb_invariances_and_autograd(orc, tr, wl):
    """Unique list (weights 2 - delta_ij) equals the ordered list; padding adds nothing; the full
    list exceeds the DF energy (E_J^DF <= E_J, gs-dft tests/unit/test_coulomb_df.py:54); autograd
    of the literal form agrees with central differences of the oracle."""
    s, pi, pj, w = _nuc_system(wl, orc, M=16, seed=7)
    E, _ = orc.exact_coulomb(s.quat, s.log_scale, s.centers, s.C, s.occ, pi, pj, w)
    po, qo, wo, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, 1e-7, None, False)
    Eo, _ = orc.exact_coulomb(s.quat, s.log_scale, s.centers, s.C, s.occ, po, qo, wo)
    assert abs(Eo - E) < 1e-12 * abs(E)
    pp, qp, wp, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, 1e-7, len(pi) + 9, True)
    Ep, _ = orc.exact_coulomb(s.quat, s.log_scale, s.centers, s.C, s.occ, pp, qp, wp)
    assert Ep == E
    la, ac = orc.product_aux(s.quat, s.log_scale, s.centers, (0.5, 1.0, 2.0, 4.0))
    fi, fj, fw, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, -1.0, None, True)
    Efull, _ = orc.exact_coulomb(s.quat, s.log_scale, s.centers, s.C, s.occ, fi, fj, fw)
    Edf = orc.dfj_energy(s.quat, s.log_scale, s.centers, s.C, s.occ, la, ac, fi, fj, fw, 1e-8)[0]
    assert Edf <= Efull * (1 + 1e-9)
    args = [_t(s.quat, True), _t(s.log_scale, True), _t(s.centers, True), _t(s.C, True)]
    Et = tr.screened_coulomb_energy(*args, _t(s.occ), _idx(pi), _idx(pj), _t(w))
    Et.backward()
    h = 1e-5
    for k, (name, arr) in enumerate((("quat", s.quat), ("log_scale", s.log_scale),
                                     ("centers", s.centers), ("C", s.C))):
        for idx in [(0, 0), (arr.shape[0] - 1, 1)]:
            up, dn = arr.copy(), arr.copy()
            up[idx] += h; dn[idx] -= h
            v = dict(quat=s.quat, log_scale=s.log_scale, centers=s.centers, C=s.C)
            v[name] = up
            eu, _ = orc.exact_coulomb(v["quat"], v["log_scale"], v["centers"], v["C"], s.occ, pi, pj, w)
            v[name] = dn
            ed, _ = orc.exact_coulomb(v["quat"], v["log_scale"], v["centers"], v["C"], s.occ, pi, pj, w)
            fd = (eu - ed) / (2 * h)
            assert abs(fd - args[k].grad[idx].item()) < 1e-6 * max(1.0, abs(fd)), (name, idx)


# ----------------------------------------------------------------------------- screened RI-K

def _exch_system(wl, orc, M=14, k=3, seed=11, eps=1e-7, n_atoms=3):
    s = wl.make_small(M, k, n_atoms=n_atoms, seed=seed)
    la, ac = orc.product_aux(s.quat, s.log_scale, s.centers, s.scales)
    pi, pj, w, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, eps, None, False)
    return s, la, ac, pi, pj, w


def test_exchange_single_orbital_is_minus_twice_dfj(orc, wl):
    """k = 1: D_P = gamma_P at occupation 1, so E_K = -gamma^T (V + lam I)^-1 gamma = -2 E_J^DF on
    the same list -- the RI-K chain against the DF-J chain, which is pinned on its own above."""
    for seed in (11, 12):
        s, la, ac, pi, pj, w = _exch_system(wl, orc, seed=seed)
        C1 = s.C[:, :1]
        EK, _ = orc.exchange_energy(s.quat, s.log_scale, s.centers, C1, la, ac, pi, pj, w, 1e-8)
        EJ = orc.dfj_energy(s.quat, s.log_scale, s.centers, C1, np.ones(1), la, ac, pi, pj, w,
                            1e-8)[0]
        assert EK < 0 and abs(EK + 2 * EJ) < 1e-11 * abs(EK)


def test_exchange_invariant_under_occupied_rotations(orc, wl):
    """E_K of a closed-shell determinant depends on span(C) only: E_K(C U) = E_K(C) for orthogonal
    U (a contraction that pairs o with itself, or drops the o != o' terms, is not invariant)."""
    s, la, ac, pi, pj, w = _exch_system(wl, orc, k=4, seed=13)
    U, _ = np.linalg.qr(np.random.default_rng(5).normal(size=(4, 4)))
    E1, D1 = orc.exchange_energy(s.quat, s.log_scale, s.centers, s.C, la, ac, pi, pj, w, 1e-8)
    E2, D2 = orc.exchange_energy(s.quat, s.log_scale, s.centers, s.C @ U, la, ac, pi, pj, w, 1e-8)
    assert abs(E1 - E2) < 1e-12 * abs(E1)
    # and D transforms as U^T D_P U
    assert rel_max(np.einsum("ao,Pab,bq->Poq", U, D1, U), D2) < 1e-12


def test_exchange_equals_density_matrix_form(orc, wl):
    """Full ordered list: the occupied form equals the density-matrix form the reference gives
    for SCF use (gs_dft/coulomb/ri.py:384-405), E_K = -1/4 sum_PQ (V + lam I)^-1_PQ Tr(Y_Q Y_P)
    with Y_P = T_P P, P = 2 C C^T, T_P[i, k] = (P|ik): a different contraction order that a
    transposed or self-paired index would break."""
    M, k = 10, 3
    s = wl.make_small(M, k, n_atoms=2, seed=17)
    la, ac = orc.product_aux(s.quat, s.log_scale, s.centers, s.scales)
    pi, pj = np.repeat(np.arange(M), M), np.tile(np.arange(M), M)
    w = np.ones(M * M)
    E, _ = orc.exchange_energy(s.quat, s.log_scale, s.centers, s.C, la, ac, pi, pj, w, 1e-8)
    T = orc.three_center_block(s.quat, s.log_scale, s.centers, la, ac, pi, pj).reshape(-1, M, M)
    P = 2.0 * s.C @ s.C.T
    Y = np.einsum("Ppr,rs->Pps", T, P)
    Wm = np.einsum("Pba,Qab->PQ", Y, Y)
    Ed = -0.25 * np.trace(np.linalg.solve(orc.aux_metric(la, ac, 1e-8), Wm))
    assert abs(E - Ed) < 1e-11 * abs(E)


def test_exchange_mask_drops_entries_and_padding(orc, wl):
    """valid is a mask (gs_dft/coulomb/ri.py:529): zero entries add nothing, so deleting them or
    appending zero-weight padding leaves E_K unchanged to the bit of the einsum order."""
    s, la, ac, pi, pj, w = _exch_system(wl, orc, seed=19)
    rng = np.random.default_rng(3)
    wm = w * (rng.uniform(size=w.shape) > 0.2)
    E1, _ = orc.exchange_energy(s.quat, s.log_scale, s.centers, s.C, la, ac, pi, pj, wm, 1e-8)
    keep = wm != 0
    E2, _ = orc.exchange_energy(s.quat, s.log_scale, s.centers, s.C, la, ac, pi[keep], pj[keep],
                                wm[keep], 1e-8)
    pp = np.concatenate([pi[keep], np.zeros(7, np.int32)])
    qp = np.concatenate([pj[keep], np.zeros(7, np.int32)])
    E3, _ = orc.exchange_energy(s.quat, s.log_scale, s.centers, s.C, la, ac, pp, qp,
                                np.concatenate([wm[keep], np.zeros(7)]), 1e-8)
    assert abs(E1 - E2) < 1e-13 * abs(E1) and abs(E2 - E3) < 1e-13 * abs(E2)


def test_exchange_literal_restatement_matches_oracle(orc, tr, wl):
    """The C-integral oracle against the torch line-by-line form (eigh three-centre block,
    occupied-chunk stream with occ_chunk smaller than k)."""
    s, la, ac, pi, pj, w = _exch_system(wl, orc, k=5, seed=23)
    wm = w * (np.random.default_rng(4).uniform(size=w.shape) > 0.1)
    E, _ = orc.exchange_energy(s.quat, s.log_scale, s.centers, s.C, la, ac, pi, pj, wm, 1e-8)
    Et = tr.screened_exchange_energy(_t(s.quat), _t(s.log_scale), _t(s.centers), _t(s.C), _t(la),
                                     _t(ac), _idx(pi), _idx(pj), _t(wm), 1e-8, chunk=64,
                                     occ_chunk=2).item()
    assert abs(E - Et) < 1e-12 * abs(E)


def test_exchange_is_exact_when_the_aux_spans_the_products(tr):
    """Isotropic splats far apart, one orbital, aux = the self-products at scale 1: every listed
    product g_i g_i is an aux function up to its norm, so the fit is exact and (with lam = 0)
    E_K = -sum_ij C_i^2 C_j^2 (ii|jj), the closed-form Gaussian Coulomb integral. A 400-node rule
    takes the three-centre quadrature error out; the metric is closed-form already."""
    rng = np.random.default_rng(41)
    M = 3
    alpha = np.exp(rng.uniform(-0.5, 0.5, M))
    quat = rng.normal(size=(M, 4))
    ls = np.repeat(np.log(alpha)[:, None], 3, 1)
    mu = np.array([[0.0, 0.0, 0.0], [30.0, 0.0, 0.0], [0.0, 40.0, 0.0]])
    C = rng.normal(size=(M, 1))
    la = np.log(2.0 * alpha)                  # det(A_i + A_i)^(1/3) = 2 alpha_i
    pi = pj = np.arange(M)
    x, wl_ = np.polynomial.legendre.leggauss(400)
    sgl = (x + 1) / 2
    table = ([float(v) for v in sgl / (1 - sgl)], [float(v) for v in (wl_ / 2) / (1 - sgl) ** 2])
    E = tr.screened_exchange_energy(_t(quat), _t(ls), _t(mu), _t(C), _t(la), _t(mu), _idx(pi),
                                    _idx(pj), _t(np.ones(M)), 0.0, table=table).item()
    A, N = tr.splat_A(_t(quat), _t(ls)), tr.splat_norm(_t(ls))
    _, _, KN = tr.full_pair_quantities(A, _t(mu), N, _idx(pi), _idx(pj))
    KN = KN.numpy()
    p = 2.0 * alpha
    ref = 0.0
    for a in range(M):
        for b in range(M):
            rho = p[a] * p[b] / (p[a] + p[b])
            T = rho * np.sum((mu[a] - mu[b]) ** 2)
            F0 = 0.5 * math.sqrt(math.pi / T) * erf(math.sqrt(T)) if T > 1e-12 else 1.0 - T / 3
            eri = KN[a] * KN[b] * 2 * math.pi ** 2.5 / (p[a] * p[b] * math.sqrt(p[a] + p[b])) * F0
            ref -= C[a, 0] ** 2 * C[b, 0] ** 2 * eri
    assert abs(E - ref) < 1e-10 * abs(ref)


# ----------------------------------------------------------------------------- long range (erf)

def test_long_range_rule_integrates_the_erf_kernel(orc):
    """The 12-node segment rule of gs_dft/integrals/dense.py:56-76 integrates the node kernel
    (2/sqrt(pi)) int_0^omega e^(-t^2 r^2) dt = erf(omega r) / r: a wrong map or weight scale fails
    at every r."""
    for om in (0.11, 0.3, 1.0):
        t, w = orc.lr_quad_table(om)
        assert np.all(np.diff(t) > 0) and t[0] > 0 and t[-1] < om
        for r in np.linspace(0.01, 3.0 / om, 50):
            q = 2.0 / math.sqrt(math.pi) * np.sum(w * np.exp(-t * t * r * r))
            assert abs(q - erf(om * r) / r) < 2e-12 * erf(om * r) / r


def _lr_metric_by_quadrature(a, A, b, B, om):
    """(s_a|erf(om r)/r|s_b) of unit-L2-normalised s-Gaussians from the Gaussian-kernel integral
    int int g_a g_b e^(-t^2 r12^2) = pi^3 / (a b)^(3/2) (rho / (rho + t^2))^(3/2)
    exp(-rho t^2 R^2 / (rho + t^2)), integrated over t in [0, om] by 400-node Gauss-Legendre."""
    NA, NB = (2 * a / math.pi) ** 0.75, (2 * b / math.pi) ** 0.75
    rho = a * b / (a + b)
    R2 = float(np.sum((np.asarray(A) - np.asarray(B)) ** 2))
    x, wl = np.polynomial.legendre.leggauss(400)
    t = 0.5 * om * (x + 1)
    f = (rho / (rho + t * t)) ** 1.5 * np.exp(-rho * t * t * R2 / (rho + t * t))
    return NA * NB * 2 / math.sqrt(math.pi) * math.pi ** 3 / (a * b) ** 1.5 * 0.5 * om * np.sum(wl * f)


def test_long_range_metric_against_the_gaussian_kernel_integral(orc):
    """ri.py:70-72's erf metric against the node integral of the Gaussian kernel (a different
    derivation: no Boys function), plus the limits omega -> infinity (the 1/r metric) and
    omega -> 0 (omega^2-scaled point charges)."""
    rng = np.random.default_rng(61)
    N = 24
    la = rng.uniform(-2.5, 2.0, N)
    cen = rng.normal(0, 2.0, (N, 3))
    cen[5] = cen[4]
    beta = np.exp(la)
    for om in (0.11, 0.3, 2.0):
        V = orc.aux_metric(la, cen, 0.0, om)
        ref = np.array([[_lr_metric_by_quadrature(beta[p], cen[p], beta[q], cen[q], om)
                         for q in range(N)] for p in range(N)])
        assert np.max(np.abs(V - ref) / np.abs(ref)) < 1e-12
        assert np.array_equal(V, V.T)
    Vfull = orc.aux_metric(la, cen)
    assert np.max(np.abs(orc.aux_metric(la, cen, 0.0, 1e7) - Vfull) / Vfull) < 1e-12
    # omega -> 0: erf(om r)/r -> 2 om / sqrt(pi), so V -> 2 om / sqrt(pi) x (charges)
    q = (2 * math.pi / beta) ** 0.75
    V0 = orc.aux_metric(la, cen, 0.0, 1e-7)
    assert np.max(np.abs(V0 / (2e-7 / math.sqrt(math.pi) * np.outer(q, q)) - 1)) < 1e-9


def test_long_range_three_centre_converges_to_the_erf_closed_form(orc, tr):
    """Isotropic pair products under the 12-node rule on [0, omega]: the (iso aux | pair) integral
    equals the textbook erf-attenuated s-s integral, sqrt(z) F0(z rho R^2) with
    z = omega^2 / (omega^2 + rho), to ~1e-15 at the omegas of range-separated hybrids (the
    reference measures ~1e-13 for its 12 nodes); the torch literal kernel under the same rule
    agrees."""
    rng = np.random.default_rng(16)
    M = 6
    alpha = np.exp(rng.uniform(-1.5, 1.0, M))
    quat = np.tile([1.0, 0, 0, 0], (M, 1))
    ls = np.repeat(np.log(alpha)[:, None], 3, 1)
    mu = rng.normal(0, 1.2, (M, 3))
    pi = np.repeat(np.arange(M), M); pj = np.tile(np.arange(M), M)
    la = rng.uniform(-1.0, 1.5, 5)
    ac = rng.normal(0, 1.5, (5, 3))
    A, Nn = orc.chart(quat, ls)
    _, P, KN = orc.pair_quantities(A, mu, Nn, pi, pj)
    beta, p = np.exp(la), alpha[pi] + alpha[pj]
    At, Nt = tr.splat_A(_t(quat), _t(ls)), tr.splat_norm(_t(ls))
    Ah_t, P_t, KN_t = tr.full_pair_quantities(At, _t(mu), Nt, _idx(pi), _idx(pj))
    for om in (0.11, 0.3):
        t, w = orc.lr_quad_table(om)
        with orc.node_rule(t, w):
            B = orc.three_center_block(quat, ls, mu, la, ac, pi, pj)
        for a_ in range(len(pi)):
            for P_ in range(len(la)):
                R = np.linalg.norm(ac[P_] - P[a_])
                red = beta[P_] * p[a_] / (beta[P_] + p[a_])
                z = om * om / (om * om + red)
                T = z * red * R * R
                F0 = 0.5 * math.sqrt(math.pi / T) * erf(math.sqrt(T)) if T > 1e-12 else 1 - T / 3
                ref = ((2 * beta[P_] / math.pi) ** 0.75 * KN[a_] * 2 * math.pi ** 2.5
                       / (beta[P_] * p[a_] * math.sqrt(beta[P_] + p[a_])) * math.sqrt(z) * F0)
                assert abs(B[P_, a_] - ref) < 1e-13 * abs(ref)
        Bt = tr.full_isobra_block(*tr.aux_quantities(_t(la), _t(ac)), Ah_t, P_t, KN_t,
                                  ([float(v) for v in t], [float(v) for v in w])).numpy()
        assert np.max(np.abs(B - Bt) / np.abs(Bt)) < 1e-12
    # the reference table is back in place afterwards
    B20 = orc.three_center_block(quat, ls, mu, la, ac, pi, pj)
    B20t = tr.full_isobra_block(*tr.aux_quantities(_t(la), _t(ac)), Ah_t, P_t, KN_t).numpy()
    assert np.max(np.abs(B20 - B20t) / np.abs(B20t)) < 1e-12


def lr_tolerance(cond):
    """Relative bound on E_K[erf] between two correct evaluations: the erf kernel is smooth, so
    its metric is far worse conditioned than the 1/r one (cond(V + lam I) ~ 1e9 at lam = 1e-8
    against ~1e4), and E_K = -tr((V + lam I)^-1 M) inherits ~cond x eps from round-off in V and M
    (measured: 1.6e-17 to 8.6e-17 x cond between the oracle and the torch literal)."""
    return max(1e-12, 1e-15 * cond)


def test_long_range_exchange_literal_matches_oracle(orc, tr, wl):
    """E_K[erf(omega r)/r]: the C-integral oracle against the torch line-by-line form (eigh
    three-centre block under the segment rule, erf metric, occupied chunks), within the
    conditioning bound; at lam = 1e-2 (cond ~1e4) that is below the 1e-10 bar."""
    s, la, ac, pi, pj, w = _exch_system(wl, orc, k=5, seed=23)
    for om in (0.11, 0.3):
        t, wq = orc.lr_quad_table(om)
        for lam in (1e-8, 1e-2):
            cond = np.linalg.cond(orc.aux_metric(la, ac, lam, om))
            E, _ = orc.exchange_energy(s.quat, s.log_scale, s.centers, s.C, la, ac, pi, pj, w,
                                       lam, omega=om)
            Et = tr.screened_exchange_energy(_t(s.quat), _t(s.log_scale), _t(s.centers),
                                             _t(s.C), _t(la), _t(ac), _idx(pi), _idx(pj), _t(w),
                                             lam, chunk=64, occ_chunk=2,
                                             table=([float(v) for v in t],
                                                    [float(v) for v in wq]),
                                             omega=om).item()
            assert abs(E - Et) < lr_tolerance(cond) * abs(E)
            if lam == 1e-2:
                assert lr_tolerance(cond) <= 1e-10
        E_full, _ = orc.exchange_energy(s.quat, s.log_scale, s.centers, s.C, la, ac, pi, pj, w,
                                        1e-8)
        assert E < 0 and abs(E) < abs(E_full)       # the long-range part of a negative energy


def test_exchange_autograd_matches_finite_differences(orc, tr, wl):
    """Autograd of the literal form against central differences of the oracle."""
    s, la, ac, pi, pj, w = _exch_system(wl, orc, M=12, k=3, seed=29)
    args = [_t(s.quat, True), _t(s.log_scale, True), _t(s.centers, True), _t(s.C, True)]
    Et = tr.screened_exchange_energy(*args, _t(la), _t(ac), _idx(pi), _idx(pj), _t(w), 1e-8)
    Et.backward()
    h = 1e-5
    base = dict(quat=s.quat, log_scale=s.log_scale, centers=s.centers, C=s.C)
    for k, name in enumerate(("quat", "log_scale", "centers", "C")):
        arr = base[name]
        for idx in [(0, 0), (arr.shape[0] - 1, 1), (5, 2)]:
            vals = []
            for sgn in (1, -1):
                v = dict(base)
                v[name] = arr.copy()
                v[name][idx] += sgn * h
                vals.append(orc.exchange_energy(v["quat"], v["log_scale"], v["centers"], v["C"],
                                                la, ac, pi, pj, w, 1e-8)[0])
            fd = (vals[0] - vals[1]) / (2 * h)
            assert abs(fd - args[k].grad[idx].item()) < 1e-6 * max(1.0, abs(fd)), (name, idx)


# ----------------------------------------------------------------------------- density on a grid

def test_grid_density_integrates_to_the_orbital_overlaps(orc, tr, wl):
    """gs_dft/screening/grid.py:52-70,88-112: on a fine Cartesian grid (the rectangle rule converges
    spectrally for Gaussians), sum_r w psi_o psi_p reproduces C^T S C with S the normalised overlap
    of the oracle (pairs.py:342-345), so the basis values, the norm and the contraction are pinned;
    in particular each splat integrates to one."""
    rng = np.random.default_rng(3)
    M = 3
    quat = rng.normal(size=(M, 4))
    ls = rng.uniform(np.log(0.6), np.log(2.0), (M, 3))
    mu = rng.normal(0, 0.5, (M, 3))
    C = rng.normal(size=(M, 2))
    h = 0.08
    ax = np.arange(-6.0, 6.0 + h / 2, h)
    X, Y, Z = np.meshgrid(ax, ax, ax, indexing="ij")
    pts = _t(np.stack([X.ravel(), Y.ravel(), Z.ravel()], 1))
    A, N = tr.splat_A(_t(quat), _t(ls)), tr.splat_norm(_t(ls))
    g, _ = tr.full_eval_block(A, _t(mu), N, pts)
    Sgrid = (g.T @ g).numpy() * h ** 3
    pi = np.repeat(np.arange(M), M); pj = np.tile(np.arange(M), M)
    S = orc.overlap_pairs(quat, ls, mu, pi, pj).reshape(M, M)
    assert np.max(np.abs(np.diag(Sgrid) - 1.0)) < 1e-10
    assert np.max(np.abs(Sgrid - S)) < 1e-10
    rho, = tr.chunked_density(_t(quat), _t(ls), _t(mu), _t(C), _t(np.ones(2)), pts, kind="lda",
                              chunk=200000)
    assert abs(rho.sum().item() * h ** 3 - np.trace(C.T @ S @ C)) < 1e-9 * np.trace(C.T @ S @ C)


def test_grid_density_gradient_and_tau_by_differences(tr, wl):
    """grad rho against central differences of rho; tau = 1/2 sum_o occ_o |grad psi_o|^2 against
    differences of psi; the GGA form (phi = (psi occ) C^T) equals the meta-GGA form
    (2 sum occ psi grad psi); chunking changes nothing."""
    s = wl.make_small(12, 3, n_atoms=2, seed=9)
    pts = _t(np.random.default_rng(1).normal(0, 2.0, (40, 3)))
    args = (_t(s.quat), _t(s.log_scale), _t(s.centers), _t(s.C), _t(s.occ))
    rho, grad = tr.chunked_density(*args, pts, kind="gga")
    rho2, grad2, tau = tr.chunked_density(*args, pts, kind="mgga", chunk=7)
    assert torch.allclose(rho, rho2, rtol=1e-14, atol=0) and rel_max(grad2.numpy(), grad.numpy()) < 1e-13
    h = 1e-5
    A, N = tr.splat_A(args[0], args[1]), tr.splat_norm(args[1])
    for d in range(3):
        e = torch.zeros(3, dtype=torch.float64); e[d] = h
        rp, = tr.chunked_density(*args, pts + e, kind="lda")
        rm, = tr.chunked_density(*args, pts - e, kind="lda")
        assert rel_max(((rp - rm) / (2 * h)).numpy(), grad[:, d].numpy()) < 1e-7
    dpsi2 = torch.zeros(pts.shape[0], s.k, dtype=torch.float64)
    for d in range(3):
        e = torch.zeros(3, dtype=torch.float64); e[d] = h
        gp, _ = tr.full_eval_block(A, args[2], N, pts + e)
        gm, _ = tr.full_eval_block(A, args[2], N, pts - e)
        dpsi2 += (((gp - gm) / (2 * h)) @ args[3]) ** 2
    tau_fd = 0.5 * (dpsi2 * args[4][None, :]).sum(1)
    assert rel_max(tau_fd.numpy(), tau.numpy()) < 1e-7
