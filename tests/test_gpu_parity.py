"""Parity of the HIP path against the CPU oracle on the same seeded inputs.

Bars: the pair list bit-exact (indices, order, weights); S within a few ulps; aux, metric,
gamma, E_J and J within 1e-10 relative (gamma ~1e-12 in practice); gradients within 1e-9
relative to the largest entry.
"""
import numpy as np
import pytest
import torch

from conftest import rel_max

pytestmark = pytest.mark.gpu

REL_E = 1e-10
REL_G = 1e-9


def _splat(g, s, grad=False):
    mk = lambda a: torch.tensor(a, device="cuda", dtype=torch.float64).requires_grad_(grad)
    return g.Splat(quat=mk(s.quat), log_scale=mk(s.log_scale), centers=mk(s.centers))


def _np(t):
    return t.detach().cpu().numpy()


SMALL = [dict(M=24, k=5, n_atoms=3, seed=1), dict(M=60, k=7, n_atoms=5, seed=2, spread=4.0),
         dict(M=200, k=9, n_atoms=8, seed=3, spread=6.0)]


def _small(wl, spec):
    spec = dict(spec)
    return wl.make_small(spec.pop("M"), spec.pop("k"), **spec)


# ----------------------------------------------------------------------------- chart / overlap

def test_chart_matches_oracle(g, wl, orc, cuda):
    s = _small(wl, SMALL[2])
    A, N = _splat(g, s).chart()
    Ao, No = orc.chart(s.quat, s.log_scale)
    assert rel_max(_np(A), Ao) < 4e-16 * 8 and rel_max(_np(N), No) < 4e-16 * 8


def test_overlap_matches_oracle_to_conditioning(g, wl, orc, cuda):
    """S = N_i N_j exp(-e) pi^1.5 / sqrt(det) is evaluated in the same operation order on both
    sides; the chart's transcendentals (exp, pow) differ by an ulp between the GPU math library
    and glibc, and that difference is amplified by the cancellation inside
    e = d . A_i (A_i + A_j)^-1 A_j d and then by exp's conditioning |e| ~ |ln S|. Most values come
    out bit-identical; the bound is 1e-13 (1 + |ln S|) relative. (The pair list itself is compared
    bit for bit in the tests below.)"""
    s = _small(wl, SMALL[2])
    M = s.M
    pi = np.repeat(np.arange(M), M).astype(np.int32)
    pj = np.tile(np.arange(M), M).astype(np.int32)
    S = _np(g.screened_overlap_pairs(_splat(g, s), torch.tensor(pi, device="cuda"),
                                     torch.tensor(pj, device="cuda")))
    So = orc.overlap_pairs(s.quat, s.log_scale, s.centers, pi, pj)
    live = So > 1e-300
    rel = np.abs(S[live] - So[live]) / So[live]
    ulps = np.abs(S - So)[live] / np.spacing(So[live])
    print(f"[overlap] ulp differences: median {np.median(ulps):.1f}, max {ulps.max():.1f}; "
          f"identical {np.mean(ulps == 0):.3f}")
    assert np.all(rel <= 1e-13 * (1.0 + np.abs(np.log(So[live]))))


# ----------------------------------------------------------------------------- pair list

def _check_list(g, s, orc, eps, unique, pad_to=None, spatial=False):
    pi, pj, v = g.neighbor_pairs(_splat(g, s), eps=eps, pad_to=pad_to, unique=unique,
                                 spatial=spatial)
    ri, rj, rw, n_sig = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, eps, pad_to, unique)
    assert np.array_equal(_np(pi), ri) and np.array_equal(_np(pj), rj)
    w = _np(v)
    if unique:
        assert v.dtype == torch.float64 and np.array_equal(w, rw)
    else:
        assert v.dtype == torch.bool and np.array_equal(w, rw != 0)
    return len(ri), n_sig


@pytest.mark.parametrize("spatial", [False, True])
@pytest.mark.parametrize("unique", [False, True])
@pytest.mark.parametrize("eps", [1e-5, 1e-7, 1e-9])
@pytest.mark.parametrize("which", [0, 1, 2])
def test_pair_list_bit_exact_small(g, wl, orc, cuda, which, eps, unique, spatial):
    s = _small(wl, SMALL[which])
    n, n_sig = _check_list(g, s, orc, eps, unique, spatial=spatial)
    assert n == n_sig == g.count_significant(_splat(g, s), eps, unique, spatial=spatial)


@pytest.mark.parametrize("spatial", [False, True])
@pytest.mark.parametrize("system", [1, 2, 3])
@pytest.mark.parametrize("eps", [1e-5, 1e-7, 1e-9])
def test_pair_list_bit_exact_benchmark_systems(g, wl, orc, cuda, system, eps, spatial):
    s = wl.make_system(system)
    print(f"[pairs] system {system} M={s.M} eps={eps} spatial={spatial}", flush=True)
    n, _ = _check_list(g, s, orc, eps, True, spatial=spatial)
    if system < 3:
        _check_list(g, s, orc, eps, False, spatial=spatial)
    print(f"[pairs] system {system}: {n} unique pairs bit-exact", flush=True)


def test_spatial_screening_on_degenerate_charts(g, wl, orc, cuda):
    """Splats whose chart bound degenerates: quaternions of norm 1e-9 and 0 (the chart then
    rotates by a non-unit quaternion, so the eigenvalue bound widens or gives up and the splat
    is a candidate for every pair), coincident centres and near-isotropic and needle-like widths:
    the spatial list still equals the oracle's."""
    s = _small(wl, SMALL[2])
    quat = s.quat.copy()
    quat[::17] *= 1e-9
    quat[5] = 0.0
    centers = s.centers.copy()
    centers[40] = centers[41]
    ls = s.log_scale.copy()
    ls[7] = [4.0, -3.5, 0.0]
    s2 = wl.System(name="degenerate", atoms=s.atoms, quat=quat, log_scale=ls, centers=centers,
                   C=s.C, occ=s.occ)
    for eps in (1e-3, 1e-7, 1e-11):
        for unique in (False, True):
            _check_list(g, s2, orc, eps, unique, spatial=True)


@pytest.mark.parametrize("spatial", [False, True])
def test_pair_list_padding_full_and_overflow(g, wl, orc, cuda, spatial):
    """gs-dft tests/unit/test_device_pairs.py:62,76,91,146 and test_pair_tricks.py:57,260; the
    spatial build falls back to the dense keep-largest rule when the list overflows its pad
    (pairs.py:290-298)."""
    s = _small(wl, SMALL[1])
    M = s.M
    for unique in (False, True):
        n, _ = _check_list(g, s, orc, 1e-7, unique, spatial=spatial)
        _check_list(g, s, orc, 1e-7, unique, pad_to=n + 37, spatial=spatial)
        _check_list(g, s, orc, 1e-7, unique, pad_to=M * M + 500, spatial=spatial)
        _check_list(g, s, orc, 1e-7, unique, pad_to=n // 2 + 1, spatial=spatial)  # keep-largest
        with pytest.raises(ValueError, match="exceed"):
            g.neighbor_pairs(_splat(g, s), eps=1e-7, pad_to=n // 3, unique=unique,
                             spatial=spatial)
    for pad in (None, M * M, M * M + 313):
        _check_list(g, s, orc, -1.0, False, pad_to=pad)
    _check_list(g, s, orc, -1.0, True)
    _check_list(g, s, orc, -1.0, False, pad_to=M * M // 2)                # eps<0, pad < M^2


@pytest.mark.parametrize("spatial", [False, True])
def test_empty_list(g, wl, cuda, spatial):
    s = wl.make_small(8, 2, n_atoms=8, spread=200.0, seed=4, width=(0.3, 0.31))
    pi, pj, v = g.neighbor_pairs(_splat(g, s), eps=0.5, unique=False, spatial=spatial)
    assert pi.shape[0] == 8 and bool(v.all())              # only the diagonal (S_ii = 1)
    pi, pj, v = g.neighbor_pairs(_splat(g, s), eps=2.0, spatial=spatial)
    assert pi.shape[0] == 0


# ----------------------------------------------------------------------------- aux / metric

def test_product_aux_and_metric_match_oracle(g, wl, orc, cuda):
    s = wl.make_system(2)
    aux = g.init_product_aux(_splat(g, s), scales=s.scales)
    la, ac = orc.product_aux(s.quat, s.log_scale, s.centers, s.scales)
    assert rel_max(_np(aux.log_alpha), la) < 1e-15 and rel_max(_np(aux.centers), ac) < 1e-14
    V = _np(g.aux_metric(aux))
    Vo = orc.aux_metric(la, ac)
    assert np.max(np.abs(V - Vo) / np.abs(Vo)) < 1e-13
    assert np.array_equal(V, V.T)


def test_product_aux_of_listed_pairs_matches_oracle(g, wl, orc, cuda):
    """init_product_aux(basis, pi, pj, valid, diagonal_only=False) (gs_dft/basis/isotropic.py:
    106-116) on a padded pair list with bool and float weights and a 20-rung scale ladder (more
    than one launch of scales), and the reference's diagonal fallbacks: diagonal_only=True, or no
    pi, give the self-product aux."""
    s = _small(wl, SMALL[1])
    basis = _splat(g, s)
    pi, pj, w = g.neighbor_pairs(basis, eps=1e-5, pad_to=None, unique=True)
    n = pi.shape[0]
    pad = torch.zeros(17, dtype=torch.int32, device="cuda")
    pi, pj = torch.cat([pi, pad]), torch.cat([pj, pad])
    w = torch.cat([w, torch.zeros(17, dtype=torch.float64, device="cuda")])
    scales = tuple(0.25 * 1.2 ** k for k in range(20))
    for valid in (w, w != 0, None):
        aux = g.init_product_aux(basis, pi, pj, valid, scales=scales, diagonal_only=False)
        vo = None if valid is None else _np(valid).astype(float)
        la, ac = orc.product_aux_pairs(s.quat, s.log_scale, s.centers, _np(pi), _np(pj), vo,
                                       scales)
        assert aux.n_basis == 20 * (n + 17)
        assert rel_max(_np(aux.log_alpha), la) < 1e-15 and rel_max(_np(aux.centers), ac) < 1e-14
    la, ac = orc.product_aux(s.quat, s.log_scale, s.centers, scales)
    for aux in (g.init_product_aux(basis, pi, pj, w, scales=scales, diagonal_only=True),
                g.init_product_aux(basis, scales=scales, diagonal_only=False)):
        assert rel_max(_np(aux.log_alpha), la) < 1e-15 and rel_max(_np(aux.centers), ac) < 1e-14


def test_refresh_with_off_diagonal_df_builds_the_self_product_aux(g, wl, orc, cuda):
    """refresh passes no pair list to init_product_aux (gs_dft/ks/energy.py:465-466), so
    df(diagonal=False) refreshes to the self-product aux, as df(diagonal=True) does."""
    s = wl.make_system(1)
    basis = _splat(g, s)
    states = [g.refresh(g.SplatDFJ(coulomb=g.df(scales=s.scales, lam=s.lam, diagonal=dg),
                                   screen=g.pairlist(s.eps, unique=True)), basis)
              for dg in (True, False)]
    assert torch.equal(states[0].aux.log_alpha, states[1].aux.log_alpha)
    assert torch.equal(states[0].aux.centers, states[1].aux.centers)
    assert torch.equal(states[0].cholV, states[1].cholV)


def test_cholesky_and_solve(g, wl, orc, cuda):
    """L L^T reproduces V + lam I to backward-stable accuracy, and the solve matches LAPACK for a
    right-hand side in the range of V (the physical case: gamma is the Coulomb projection of a
    density). cond(V + lam I) is ~3e11 here, so a random right-hand side would only be
    reproducible to ~cond * eps between any two factorisations."""
    s = wl.make_system(1)
    aux = g.init_product_aux(_splat(g, s), scales=s.scales)
    L = g.aux_cholesky(aux, 1e-8)
    Ln = _np(L)
    la, ac = orc.product_aux(s.quat, s.log_scale, s.centers, s.scales)
    V = orc.aux_metric(la, ac, 1e-8)
    N = V.shape[0]
    print(f"[solve] N={N} cond(V+lam I) = {np.linalg.cond(V):.3e}")
    assert np.all(np.triu(Ln, 1) == 0)
    assert rel_max(Ln @ Ln.T, V) < 8 * N * np.finfo(float).eps
    x = np.random.default_rng(0).normal(size=N)
    gam = torch.tensor(V @ x, device="cuda")
    E = g.df_coulomb_solve(gam, aux, cholV=L).item()
    En = 0.5 * (V @ x) @ np.linalg.solve(V, V @ x)
    assert abs(E - En) < 1e-10 * abs(En)


@pytest.mark.parametrize("system,omega", [(1, 0.0), (2, 0.0), (2, 0.4)])
def test_aux_cholesky_equals_metric_then_factor(g, wl, cuda, system, omega):
    """gsdft_aux_cholesky forms only the metric's lower triangle (zeros above it) in the factor's
    buffer and factors it in place; the factorisation reads only that triangle, so the factor is
    bit-identical to gsdft_aux_metric's full V factored by gsdft_cholesky (1/r and erf kernels)."""
    from gs_dft_amd import _lib, ri as _ri
    s = wl.make_system(system)
    aux = g.init_product_aux(_splat(g, s), scales=s.scales)
    N = aux.n_basis
    print(f"[aux_cholesky] system={system} N={N} omega={omega}", flush=True)
    lam = 1e-8 if omega == 0.0 else 1e-2
    L = g.aux_cholesky(aux, lam, omega or None)
    V = _ri.aux_metric(aux, omega or None, lam=lam)
    Lb = _lib.lib()
    ws = _lib.workspace(_lib.size_query(Lb.gsdft_metric_workspace_size, N), V.device)
    _lib.check(Lb.gsdft_cholesky(N, _lib.ptr(V), _lib.ptr(ws), ws.numel(), _lib.stream()), "chol")
    assert torch.equal(L, V)
    assert not torch.any(torch.triu(L, 1))


@pytest.mark.parametrize("N", [1, 100, 1000, 1024, 2500, 3137, 4500])
def test_blocked_cholesky_matches_lapack(g, cuda, N):
    """The blocked factorisation (2048-row panels, 128-row substitution blocks, FP64 MFMA
    updates in 128 x 128 tiles; partial last panel, block and tiles, widths not a multiple of 16)
    against LAPACK on a well-conditioned SPD matrix; the strict upper triangle is zeroed. A matrix
    made indefinite inside a later panel reports the failing leading minor of the whole matrix."""
    from gs_dft_amd import _lib
    rng = np.random.default_rng(N)
    A = rng.normal(size=(N, N)) / np.sqrt(N)
    V = A @ A.T + np.eye(N)
    print(f"[cholesky] N={N}", flush=True)
    Vd = torch.tensor(V, device="cuda")
    Lb = _lib.lib()
    ws = _lib.workspace(_lib.size_query(Lb.gsdft_metric_workspace_size, N), Vd.device)
    _lib.check(Lb.gsdft_cholesky(N, _lib.ptr(Vd), _lib.ptr(ws), ws.numel(), _lib.stream()), "chol")
    Ln = _np(Vd)
    err = rel_max(Ln, np.linalg.cholesky(V))
    print(f"[cholesky] N={N} L rel-to-max {err:.2e}")
    assert err < 1e-12
    assert np.all(np.triu(Ln, 1) == 0)
    if N > 1100:
        bad = 1100                                 # inside the second panel
        Vb = V.copy()
        Vb[bad, bad] = -1.0
        Vd = torch.tensor(Vb, device="cuda")
        with pytest.raises(torch.linalg.LinAlgError, match=f"leading minor {bad + 1} "):
            _lib.check(Lb.gsdft_cholesky(N, _lib.ptr(Vd), _lib.ptr(ws), ws.numel(),
                                         _lib.stream()), "chol")


@pytest.mark.parametrize("N,offset", [(1, 0), (64, 0), (127, 0), (128, 0), (129, 0), (192, 0),
                                      (193, 0), (256, 0), (257, 0), (300, 0), (1000, 0),
                                      (1000, 1), (2561, 0), (4096, 0), (8193, 0)])
def test_blocked_solves_match_lapack(g, cuda, N, offset):
    """The blocked substitutions (128-column blocks, one launch per block, each also solving the
    next block: next blocks of 1, 64 or 65 rows, partial last block of 1 row at 8193, steps with no
    rows past the next block) against LAPACK's triangular solves with the same factor:
    d = L^-T L^-1 gamma and E = gamma.d / 2, for a well-conditioned factor (cond(L) ~ 1e2), so the
    two agree to a few ulp times cond. offset = 1 places the factor 8 bytes past a 16-byte
    boundary (no paired loads)."""
    from scipy.linalg import solve_triangular
    from gs_dft_amd import ri as _ri
    rng = np.random.default_rng(N)
    if N <= 4096:
        A = rng.normal(size=(N, N)) / np.sqrt(N)
        Ln = np.linalg.cholesky(A @ A.T + np.eye(N))
    else:                                   # a unit-diagonal factor with small random entries
        Ln = rng.uniform(-1.0, 1.0, size=(N, N))
        for i0 in range(0, N, 1024):        # in place, by row blocks
            blk = Ln[i0:i0 + 1024]
            blk *= 0.5 / N
            blk[:] = np.tril(blk, i0 - 1)
        Ln[np.diag_indices(N)] = 1.0
    Ln[np.diag_indices(N)] *= rng.uniform(0.5, 2.0, size=N)
    gam = rng.normal(size=N)
    y = solve_triangular(Ln, gam, lower=True)
    dn = solve_triangular(Ln.T, y, lower=False)
    print(f"[solve] N={N} offset={offset}", flush=True)
    buf = torch.empty(N * N + offset, dtype=torch.float64, device="cuda")
    Ld = buf[offset:].view(N, N)
    Ld.copy_(torch.from_numpy(Ln))
    assert Ld.data_ptr() % 16 == 8 * offset
    d, E = _ri._cho_solve(Ld, torch.tensor(gam, device="cuda"), True)
    err = rel_max(_np(d), dn)
    print(f"[solve] N={N} d rel-to-max {err:.2e}")
    assert err < 1e-12
    assert abs(E.item() - 0.5 * gam @ dn) < 1e-12 * abs(0.5 * gam @ dn)


# ----------------------------------------------------------------------------- gamma / E_J / grads

def _problem(wl, orc, s, eps=None, unique=True):
    eps = s.eps if eps is None else eps
    la, ac = orc.product_aux(s.quat, s.log_scale, s.centers, s.scales)
    pi, pj, w, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, eps, None, unique)
    return la, ac, pi, pj, w


@pytest.mark.parametrize("which", [0, 1, 2])
def test_gamma_matches_oracle_small(g, wl, orc, cuda, which):
    s = _small(wl, SMALL[which])
    la, ac, pi, pj, w = _problem(wl, orc, s)
    aux = g.IsotropicSplat(log_alpha=la, centers=ac)
    gam = _np(g.df_coulomb_gamma_screened(_splat(g, s), torch.tensor(s.C, device="cuda"),
                                          s.occ, aux, pi, pj, valid=w))
    go = orc.gamma(s.quat, s.log_scale, s.centers, s.C, s.occ, la, ac, pi, pj, w)
    print(f"[gamma] M={s.M} n={len(pi)} N={len(la)} rel {rel_max(gam, go):.2e}")
    assert rel_max(gam, go) < 1e-12


def _energy_grads(g, s, la, ac, pi, pj, w, lam, pad_to=None):
    basis = _splat(g, s, grad=True)
    C = torch.tensor(s.C, device="cuda", dtype=torch.float64, requires_grad=True)
    aux = g.IsotropicSplat(log_alpha=la, centers=ac)
    L = g.aux_cholesky(aux, lam)
    if pad_to is not None:
        extra = pad_to - len(pi)
        pi = np.concatenate([pi, np.zeros(extra, np.int32)])
        pj = np.concatenate([pj, np.zeros(extra, np.int32)])
        w = np.concatenate([w, np.zeros(extra)])
    E = g.df_coulomb_energy_screened(basis, C, s.occ, aux, pi, pj, lam=lam, valid=w, cholV=L)
    E.backward()
    return (E.item(), _np(basis.quat.grad), _np(basis.log_scale.grad), _np(basis.centers.grad),
            _np(C.grad))


@pytest.mark.parametrize("case", ["small0", "small1", "system1", "system2"])
def test_energy_and_gradients_match_oracle(g, wl, orc, cuda, case):
    s = _small(wl, SMALL[int(case[-1])]) if case.startswith("small") else wl.make_system(int(case[-1]))
    la, ac, pi, pj, w = _problem(wl, orc, s)
    print(f"[dfj] {case}: M={s.M} n={len(pi)} N={len(la)} k={s.k}", flush=True)
    got = _energy_grads(g, s, la, ac, pi, pj, w, s.lam)
    ref = orc.dfj_grad(s.quat, s.log_scale, s.centers, s.C, s.occ, la, ac, pi, pj, w, s.lam)
    rel = abs(got[0] - ref[0]) / abs(ref[0])
    print(f"[dfj] {case}: E_J gpu {got[0]:.15e} oracle {ref[0]:.15e} rel {rel:.2e}")
    assert rel < REL_E
    for name, a, b in zip(("quat", "log_scale", "centers", "C"), got[1:], ref[2:]):
        err = rel_max(a, b)
        print(f"[dfj] {case}: d{name} rel-to-max {err:.2e}")
        assert err < REL_G


def test_node_screen_far_apart_matches_oracle(g, wl, orc, cuda):
    """Atoms spread over 50 Bohr: most waves leave the 20-node loop early (node terms below
    e^-46 of their prefactor), yet gamma, E_J and every gradient match the oracle's full
    20-node sums."""
    from gs_dft_amd import _lib
    s = wl.make_small(320, 6, n_atoms=10, seed=7, spread=25.0)
    la, ac, pi, pj, w = _problem(wl, orc, s)
    aux = g.IsotropicSplat(log_alpha=la, centers=ac)
    _lib.profile_enable(True)
    try:
        for kid in (_lib.PROF_GAMMA_FWD, _lib.PROF_GAMMA_BWD):
            _lib.profile_read_work(kid, reset=True)
        gam = _np(g.df_coulomb_gamma_screened(_splat(g, s), torch.tensor(s.C, device="cuda"),
                                              s.occ, aux, pi, pj, valid=w))
        fwd_nodes = _lib.profile_read_work(_lib.PROF_GAMMA_FWD, reset=True)
        got = _energy_grads(g, s, la, ac, pi, pj, w, s.lam)
        bwd_nodes = _lib.profile_read_work(_lib.PROF_GAMMA_BWD, reset=True)
    finally:
        _lib.profile_enable(False)
    full = 20 * len(la) * len(pi)
    print(f"[screen] M={s.M} n={len(pi)} N={len(la)}: nodes evaluated fwd {fwd_nodes / full:.3f} "
          f"bwd {bwd_nodes / full:.3f} of all")
    assert 0 < fwd_nodes < 0.9 * full and 0 < bwd_nodes < 0.9 * full
    go = orc.gamma(s.quat, s.log_scale, s.centers, s.C, s.occ, la, ac, pi, pj, w)
    print(f"[screen] gamma rel {rel_max(gam, go):.2e}")
    assert rel_max(gam, go) < 1e-12
    ref = orc.dfj_grad(s.quat, s.log_scale, s.centers, s.C, s.occ, la, ac, pi, pj, w, s.lam)
    rel = abs(got[0] - ref[0]) / abs(ref[0])
    print(f"[screen] E_J rel {rel:.2e}")
    assert rel < REL_E
    for name, a, b in zip(("quat", "log_scale", "centers", "C"), got[1:], ref[2:]):
        err = rel_max(a, b)
        print(f"[screen] d{name} rel-to-max {err:.2e}")
        assert err < REL_G


def test_J_on_the_pair_list_matches_oracle(g, wl, orc, cuda):
    s = _small(wl, SMALL[1])
    la, ac, pi, pj, w = _problem(wl, orc, s)
    aux = g.IsotropicSplat(log_alpha=la, centers=ac)
    J = _np(g.coulomb_pairs(_splat(g, s), torch.tensor(s.C, device="cuda"), s.occ, aux, pi, pj,
                            lam=s.lam, valid=w))
    ref = orc.dfj_grad(s.quat, s.log_scale, s.centers, s.C, s.occ, la, ac, pi, pj, w, s.lam)
    assert rel_max(J, ref[1]) < REL_E


def test_general_cotangent_of_gamma(g, wl, orc, cuda):
    """Reverse of gamma alone for d(sum gamma^2) (gs-dft tests/unit/test_pair_tricks.py:81)."""
    s = _small(wl, SMALL[0])
    la, ac, pi, pj, w = _problem(wl, orc, s)
    basis = _splat(g, s, grad=True)
    C = torch.tensor(s.C, device="cuda", dtype=torch.float64, requires_grad=True)
    aux = g.IsotropicSplat(log_alpha=la, centers=ac)
    gam = g.df_coulomb_gamma_screened(basis, C, s.occ, aux, pi, pj, valid=w)
    (gam ** 2).sum().backward()
    go = orc.gamma(s.quat, s.log_scale, s.centers, s.C, s.occ, la, ac, pi, pj, w)
    ref = orc.gamma_vjp(s.quat, s.log_scale, s.centers, s.C, s.occ, la, ac, pi, pj, w, 2 * go)
    for a, b in zip((basis.quat.grad, basis.log_scale.grad, basis.centers.grad, C.grad), ref[1:]):
        assert rel_max(_np(a), b) < REL_G


def test_unique_equals_ordered_and_padding_is_exact(g, wl, orc, cuda):
    """gs-dft tests/unit/test_pair_tricks.py:81,107 on the GPU path: the unique list reproduces
    the ordered one, and appended padding (weight 0) changes nothing."""
    s = _small(wl, SMALL[1])
    la, ac, ui, uj, uw = _problem(wl, orc, s, unique=True)
    _, _, oi, oj, ow = _problem(wl, orc, s, unique=False)
    eu = _energy_grads(g, s, la, ac, ui, uj, uw, s.lam)
    eo = _energy_grads(g, s, la, ac, oi, oj, ow, s.lam)
    ep = _energy_grads(g, s, la, ac, ui, uj, uw, s.lam, pad_to=2 * len(ui) + 100)
    assert abs(eu[0] - eo[0]) < 1e-10 * abs(eo[0])
    assert eu[0] == ep[0]
    for a, b, c in zip(eu[1:], eo[1:], ep[1:]):
        assert rel_max(a, b) < 1e-9 and np.array_equal(a, c)


def test_results_are_deterministic(g, wl, orc, cuda):
    s = _small(wl, SMALL[2])
    la, ac, pi, pj, w = _problem(wl, orc, s)
    a = _energy_grads(g, s, la, ac, pi, pj, w, s.lam)
    b = _energy_grads(g, s, la, ac, pi, pj, w, s.lam)
    assert a[0] == b[0] and all(np.array_equal(x, y) for x, y in zip(a[1:], b[1:]))


def test_plugin_surface_end_to_end(g, wl, orc, cuda):
    """df() + pairlist() + refresh() + ScreenedProductDFCoulomb.energy, as a trainer calls them
    (gs_dft/ks/train.py:355-382), against the oracle."""
    s = wl.make_system(1)
    basis = _splat(g, s, grad=True)
    C = torch.tensor(s.C, device="cuda", dtype=torch.float64, requires_grad=True)
    ks = g.SplatDFJ(coulomb=g.df(scales=s.scales, lam=s.lam),
                    screen=g.pairlist(s.eps, unique=True, skip_pad=True))
    n0 = g.neighbor_pairs(basis, eps=s.eps, unique=True)[0].shape[0]
    state = g.refresh(ks, basis, pad_to=g.train_pad_to(ks.screen, n0))
    assert state.pairs[0].shape[0] == 2 * n0 and state.cholV is not None
    state2 = g.refresh(ks, basis, like=state)
    assert state2.pairs[0].shape[0] == 2 * n0
    E_J, E_K = ks.coulomb.energy(basis, C, None, torch.tensor(s.occ, device="cuda"), state)
    assert E_K.item() == 0.0
    E_J.backward()
    la, ac, pi, pj, w = _problem(wl, orc, s)
    ref = orc.dfj_grad(s.quat, s.log_scale, s.centers, s.C, s.occ, la, ac, pi, pj, w, s.lam)
    assert abs(E_J.item() - ref[0]) < REL_E * abs(ref[0])
    for a, b in zip((basis.quat, basis.log_scale, basis.centers, C), ref[2:]):
        assert rel_max(_np(a.grad), b) < REL_G


def test_system3_sampled_gamma_and_directional_derivative(g, wl, orc, cuda):
    """Alkane (M=2000, N_aux=8000): gamma on a sample of aux functions against the oracle, and
    the gradient's directional derivative against central differences of the GPU energy."""
    s = wl.make_system(3)
    basis = _splat(g, s)
    ks = g.SplatDFJ(coulomb=g.df(scales=s.scales, lam=s.lam), screen=g.pairlist(s.eps, unique=True))
    state = g.refresh(ks, basis)
    pi, pj, w = (_np(t) for t in state.pairs)
    C = torch.tensor(s.C, device="cuda")
    gam = _np(g.df_coulomb_gamma_screened(basis, C, s.occ, state.aux, state.pairs[0],
                                          state.pairs[1], valid=state.pairs[2],
                                          index=state.pair_index))
    rng = np.random.default_rng(0)
    sel = np.sort(rng.choice(len(gam), 48, replace=False))
    la, ac = _np(state.aux.log_alpha), _np(state.aux.centers)
    go = orc.gamma(s.quat, s.log_scale, s.centers, s.C, s.occ, la[sel], ac[sel], pi, pj, w)
    print(f"[system3] n={len(pi)} sampled gamma rel {rel_max(gam[sel], go):.2e}", flush=True)
    assert rel_max(gam[sel], go) < 1e-12
    b2 = _splat(g, s, grad=True)
    Cg = C.clone().requires_grad_()
    E = ks(g.SplatModel(basis=b2, C=Cg, occupations=torch.tensor(s.occ, device="cuda")), state)
    E.backward()
    dirs = [torch.randn_like(t) for t in (b2.quat, b2.log_scale, b2.centers, Cg)]
    dd = sum((t.grad * d).sum().item() for t, d in zip((b2.quat, b2.log_scale, b2.centers, Cg), dirs))
    h = 1e-5

    def e_at(sign):
        with torch.no_grad():
            b = g.Splat(quat=b2.quat + sign * h * dirs[0], log_scale=b2.log_scale + sign * h * dirs[1],
                        centers=b2.centers + sign * h * dirs[2])
            return ks(g.SplatModel(basis=b, C=Cg + sign * h * dirs[3],
                                   occupations=torch.tensor(s.occ, device="cuda")), state).item()
    fd = (e_at(1) - e_at(-1)) / (2 * h)
    print(f"[system3] directional derivative {dd:.10e} vs central difference {fd:.10e}")
    assert abs(fd - dd) < 1e-6 * max(1.0, abs(dd))


def test_system4_directional_derivative(g, wl, orc, cuda):
    """The 300-atom CH2 globule (M = 12000, N_aux = 48000, k = 600: 64-bit offsets in the factor and
    the solves, several slabs and Cholesky panels): the gradient's directional derivative through
    the plugin surface against central differences of the GPU energy (element-level parity at
    this size is in test_gpu_fullsize.py)."""
    s = wl.make_system(4)
    basis = _splat(g, s)
    ks = g.SplatDFJ(coulomb=g.df(scales=s.scales, lam=s.lam), screen=g.pairlist(s.eps, unique=True))
    state = g.refresh(ks, basis)
    C = torch.tensor(s.C, device="cuda")
    print(f"[system4] n={state.pairs[0].shape[0]} N={state.aux.n_basis}", flush=True)
    b2 = _splat(g, s, grad=True)
    Cg = C.clone().requires_grad_()
    occ = torch.tensor(s.occ, device="cuda")
    E = ks(g.SplatModel(basis=b2, C=Cg, occupations=occ), state)
    E.backward()
    leaves = (b2.quat, b2.log_scale, b2.centers, Cg)
    gen = torch.Generator(device="cpu").manual_seed(44)
    dirs = [torch.randn(t.shape, generator=gen, dtype=torch.float64).cuda() for t in leaves]
    dd = sum((t.grad * d).sum().item() for t, d in zip(leaves, dirs))
    h = 1e-5

    def e_at(sign):
        with torch.no_grad():
            b = g.Splat(quat=b2.quat + sign * h * dirs[0], log_scale=b2.log_scale + sign * h * dirs[1],
                        centers=b2.centers + sign * h * dirs[2])
            return ks(g.SplatModel(basis=b, C=Cg + sign * h * dirs[3], occupations=occ),
                      state).item()
    fd = (e_at(1) - e_at(-1)) / (2 * h)
    print(f"[system4] E {E.item():.12e}: directional derivative {dd:.10e} vs central difference "
          f"{fd:.10e}")
    assert abs(fd - dd) < 1e-6 * max(1.0, abs(dd))
