"""Full-size parity of the HIP path against the CPU oracle at the three largest benchmark systems.

The reference checks its device pair list element for element against a host build
(gs-dft tests/unit/test_device_pairs.py:50) and its screened gradients against the unscreened
ones (tests/unit/test_screening.py:167); these are the same checks at the benchmark sizes:

* the pair list bit for bit (indices, order, weights) at the 300- and 700-atom globules, with a
  knife-edge audit of the threshold on every benchmark system;
* gradients per splat: a splat's rows of dE/d(quat, log_scale, centers, C) depend only on the list
  entries that contain it, so the oracle's reverse pass over just those entries, driven by the
  GPU's own d = (V + lam I)^-1 gamma, reproduces those rows exactly; 8 random splats per case,
  each row within 1e-9 of its largest entry, and J on those entries within 1e-10;
* the product aux against the oracle's at full size, and 66 full rows of the metric (64 random,
  the first and the last) elementwise within 1e-13 of the oracle's metric of the same aux and
  within 3e-12 of the oracle's metric of its own aux (measured up to 8e-13 at the 700-atom
  globule); the oracle's gamma rows and reverse pass run on the oracle's own aux, not the GPU's
  (the two aux differ by a few ulps times the chart's condition number, which every comparison
  through them carries);
* gamma on sampled aux rows, elementwise within 1e-12;
* the solve's normwise backward error on the oracle's metric rows, within 1e-12;
* E_J: against 1/2 gamma_o . (V_o + lam I)^-1 gamma_o computed entirely on the CPU (the oracle's
  whole gamma_o and metric V_o, LAPACK's factorisation) where the CPU can afford it (C20H42 at
  every screening threshold); at the globules, where the oracle's whole gamma would take hours of
  CPU, E_J = 1/2 gamma . d is pinned through (a) the sampled gamma rows, (b) the adjoint identity
  v . gamma = sum_a q_a J_a(v) between the forward and the reverse kernels for a random v, (c) the
  backward error above and (d) the normwise backward error of the solve against the whole metric
  built afresh on the GPU.

cond(V + lam I) is estimated per system (power and inverse iteration) and printed beside the
E_J figures.
"""
import numpy as np
import pytest
import torch

from conftest import rel_max

pytestmark = pytest.mark.gpu

REL_E = 1e-10
REL_G = 1e-9


def _np(t):
    return t.detach().cpu().numpy()


def _splat(g, s):
    mk = lambda a: torch.tensor(a, device="cuda", dtype=torch.float64)
    return g.Splat(quat=mk(s.quat), log_scale=mk(s.log_scale), centers=mk(s.centers))


# ----------------------------------------------------------------------------- pair list

_ORACLE_LISTS = {}


def _oracle_list(orc, s, unique):
    key = (s.name, s.eps, unique)
    if key not in _ORACLE_LISTS:
        _ORACLE_LISTS[key] = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, s.eps, None,
                                                unique)
    return _ORACLE_LISTS[key]


@pytest.mark.parametrize("system,unique,spatial", [(4, True, False), (4, True, True),
                                                   (4, False, True), (5, True, False),
                                                   (5, True, True)])
def test_pair_list_bit_exact_globules(g, wl, orc, cuda, system, unique, spatial):
    """The 300-atom (7.2e7 / 1.4e8 candidates) and 700-atom (2.0e8 candidates) globules at
    eps = 1e-7: the GPU list, from the dense scan and from the spatial candidates, equals the
    oracle's element for element."""
    s = wl.make_system(system)
    print(f"[pairs] system {system} M={s.M} eps={s.eps} unique={unique} spatial={spatial}",
          flush=True)
    pi, pj, v = g.neighbor_pairs(_splat(g, s), eps=s.eps, unique=unique, spatial=spatial)
    ri, rj, rw, n_sig = _oracle_list(orc, s, unique)
    assert len(ri) == n_sig == pi.shape[0]
    assert np.array_equal(_np(pi), ri) and np.array_equal(_np(pj), rj)
    if unique:
        assert np.array_equal(_np(v), rw)
    else:
        assert bool(v.all())
    print(f"[pairs] system {system}: {len(ri)} pairs bit-exact", flush=True)


def test_spatial_equals_dense_at_60k_splats(g, wl, cuda):
    """A 2100-atom globule with M = 60000 splats (1.8e9 unique candidates, beyond the oracle's
    reach in a test): the spatial build equals the dense scan bit for bit, and both counts
    agree."""
    s = wl.make_globule2100()
    basis = _splat(g, s)
    print(f"[pairs] {s.name} M={s.M} eps={s.eps}", flush=True)
    a = g.neighbor_pairs(basis, eps=s.eps, unique=True, spatial=True)
    b = g.neighbor_pairs(basis, eps=s.eps, unique=True, spatial=False)
    assert all(torch.equal(x, y) for x, y in zip(a, b))
    print(f"[pairs] {s.name}: {a[0].shape[0]} unique pairs, spatial == dense", flush=True)


@pytest.mark.parametrize("system,eps", [(3, 1e-5), (3, 1e-7), (3, 1e-9), (4, 1e-7), (5, 1e-7)])
def test_threshold_knife_edge_audit(g, wl, orc, cuda, system, eps):
    """No candidate's |S| lies within 1e-12 of eps (relative), so the few-ulp differences between
    the GPU's and glibc's exp/pow cannot move a pair across the threshold; the smallest margin
    is printed."""
    s = wl.make_system(system, eps=eps)
    n_close, gap = orc.screen_margin(s.quat, s.log_scale, s.centers, eps, True, rel_tol=1e-12)
    n10, _ = orc.screen_margin(s.quat, s.log_scale, s.centers, eps, True, rel_tol=1e-10)
    print(f"[knife-edge] system {system} eps {eps:g}: smallest ||S| - eps| / eps = {gap:.3e}; "
          f"{n_close} candidates within 1e-12, {n10} within 1e-10", flush=True)
    assert n_close == 0


# ----------------------------------------------------------------------------- E_J and gradients

def _cond_estimate(V, d_solve, iters=60):
    """(lambda_max, lambda_min) of the SPD matrix V by power iteration and inverse iteration
    (d_solve(x) = V^-1 x)."""
    gen = torch.Generator(device="cpu").manual_seed(0)
    x = torch.randn(V.shape[0], generator=gen, dtype=torch.float64).cuda()
    x /= x.norm()
    lmax = 0.0
    for _ in range(iters):
        y = torch.mv(V, x)
        lmax = float(y.norm())
        x = y / lmax
    x = torch.randn(V.shape[0], generator=gen, dtype=torch.float64).cuda()
    x /= x.norm()
    inv = 0.0
    for _ in range(iters):
        y = d_solve(x)
        inv = float(y.norm())
        x = y / inv
    return lmax, 1.0 / inv


def _splat_rows_parity(orc, s, la, ac, pin, pjn, wn, d, got, J, n_splats, seed, tag):
    """Oracle reverse pass over the entries that contain n_splats random splats, with the GPU's
    own d as the cotangent, against those splats' gradient rows and the entries' J."""
    rng = np.random.default_rng(seed)
    splats = np.sort(rng.choice(s.M, n_splats, replace=False))
    live = wn != 0
    idx = np.nonzero(live & (np.isin(pin, splats) | np.isin(pjn, splats)))[0]
    print(f"[{tag}] splats {splats.tolist()}: {len(idx)} list entries x {len(la)} aux", flush=True)
    ref = orc.gamma_vjp(s.quat, s.log_scale, s.centers, s.C, s.occ, la, ac, pin[idx], pjn[idx],
                        wn[idx], d)
    errJ = rel_max(J[idx], ref[0])
    print(f"[{tag}] J on those entries rel-to-max {errJ:.2e}", flush=True)
    assert errJ < REL_E
    worst = 0.0
    for name, a, b in zip(("quat", "log_scale", "centers", "C"), got, ref[1:]):
        for m in splats:
            scale = np.max(np.abs(b[m]))
            err = float(np.max(np.abs(a[m] - b[m])) / scale) if scale > 0 else float(np.max(np.abs(a[m])))
            worst = max(worst, err)
            assert err < REL_G, (name, int(m), err)
    print(f"[{tag}] gradient rows of {n_splats} splats: worst rel-to-row-max {worst:.2e}",
          flush=True)


@pytest.mark.parametrize("system,eps", [(3, 1e-5), (3, 1e-7), (3, 1e-9), (4, 1e-7), (5, 1e-7)])
def test_energy_gamma_and_gradient_rows_full_size(g, wl, orc, cuda, system, eps):
    from gs_dft_amd import ri as _ri
    from gs_dft_amd import screening as _scr
    tag = f"system {system} eps {eps:g}"
    s = wl.make_system(system, eps=eps)
    basis = _splat(g, s)
    ks = g.SplatDFJ(coulomb=g.df(scales=s.scales, lam=s.lam), screen=g.pairlist(eps, unique=True))
    state = g.refresh(ks, basis)
    pi, pj, w = state.pairs
    N = state.aux.n_basis
    C = torch.tensor(s.C, device="cuda")
    print(f"[{tag}] M={s.M} N_aux={N} k={s.k} n={pi.shape[0]}", flush=True)
    # the calls _EnergyFn makes: gamma, the solve with the energy, the reverse with dE/dgamma = d
    x = _ri._Inputs(basis, C, s.occ, state.aux, pi, pj, w, state.pair_index)
    gam = _ri._gamma_forward(x)
    d, E = _ri._cho_solve(state.cholV, gam, True)
    J, dq, dl, dc, dC = _ri._gamma_vjp(x, d, None)
    torch.cuda.synchronize()
    E = E.item()
    gam_n, d_n, J_n = _np(gam), _np(d), _np(J)
    got = [_np(t) for t in (dq, dl, dc, dC)]
    pin, pjn, wn = _np(pi), _np(pj), _np(w)
    # the aux the refresh built against the oracle's product aux at full size
    # (gs_dft/basis/isotropic.py:81-116); everything the oracle computes below uses its own aux
    la_o, ac_o = orc.product_aux(s.quat, s.log_scale, s.centers, s.scales)
    la_g, ac_g = _np(state.aux.log_alpha), _np(state.aux.centers)
    err_la = float(np.max(np.abs(la_g - la_o)))        # log_alpha: relative error of alpha
    err_ac = rel_max(ac_g, ac_o)
    print(f"[{tag}] aux ({N} functions) vs oracle: alpha rel {err_la:.2e}, centres "
          f"{err_ac:.2e} rel-to-max", flush=True)
    # E_J is the scaled dot of the solve's own outputs
    assert abs(E - 0.5 * float(np.dot(gam_n, d_n))) < 1e-13 * abs(E)
    # gamma: every row at C20H42, sampled rows at the globules, from the oracle's own aux
    rng = np.random.default_rng(system * 10 + int(-np.log10(eps)))
    sel = np.arange(N) if system == 3 else np.sort(rng.choice(N, 32, replace=False))
    go = orc.gamma(s.quat, s.log_scale, s.centers, s.C, s.occ, la_o[sel], ac_o[sel], pin, pjn,
                   wn)
    err = float(np.max(np.abs(gam_n[sel] - go) / np.abs(go)))
    print(f"[{tag}] {len(sel)} gamma rows: max elementwise rel {err:.2e}", flush=True)
    # the metric: 64 random full rows (and the first and last) against the oracle's
    # (gs_dft/coulomb/ri.py:63-76,267-275 with shift_diag), on the oracle's aux and, to isolate
    # the metric kernel, on the GPU's
    V = _ri.aux_metric(state.aux, lam=s.lam)
    rows = np.unique(np.concatenate([[0, N - 1], rng.choice(N, 64, replace=False)]))
    Vo_rows = orc.aux_metric_rows(la_o, ac_o, rows, s.lam)
    Vk_rows = orc.aux_metric_rows(la_g, ac_g, rows, s.lam)
    Vg_rows = _np(V[torch.tensor(rows, device="cuda")])
    err_v = float(np.max(np.abs(Vg_rows - Vo_rows) / np.abs(Vo_rows)))
    err_vk = float(np.max(np.abs(Vg_rows - Vk_rows) / np.abs(Vk_rows)))
    print(f"[{tag}] {len(rows)} metric rows x {N}: max elementwise rel {err_v:.2e} (on the "
          f"GPU's aux {err_vk:.2e})", flush=True)
    # the solve's normwise backward error on the oracle's rows: (V_o d - gamma)[rows]
    r_o = Vo_rows @ d_n - gam_n[rows]
    eta_o = float(np.max(np.abs(r_o))) / (float(np.max(np.abs(Vo_rows).sum(1)))
                                          * float(np.max(np.abs(d_n))) + float(np.max(np.abs(gam_n))))
    print(f"[{tag}] solve backward error on the oracle's metric rows {eta_o:.2e}", flush=True)
    # The aux centres are solve3(2A, 2A mu) as in the reference (isotropic.py:112), so the GPU's
    # and the oracle's differ by a few ulps times cond(A) <= 100; every figure above carries that
    # difference, the metric kernel alone (Vk) does not.
    assert err_la < 1e-13 and err_ac < 1e-13
    assert err_vk < 1e-13 and err_v < 3e-12
    assert err < 1e-12
    assert eta_o < 1e-12
    # per-splat gradient rows and J, the oracle's reverse pass on its own aux
    _splat_rows_parity(orc, s, la_o, ac_o, pin, pjn, wn, d_n, got, J_n, 8, system * 100 + 7,
                       tag)
    lmax, lmin = _cond_estimate(V, lambda v: _ri._cho_solve(state.cholV, v, False)[0])
    print(f"[{tag}] cond(V + lam I) ~ {lmax / lmin:.3e} (lambda_max {lmax:.3e}, "
          f"lambda_min {lmin:.3e})", flush=True)
    if system == 3:
        # E_J entirely from the oracle: its whole gamma, its metric and a LAPACK factorisation
        from scipy.linalg import cho_factor, cho_solve
        Vo = orc.aux_metric(la_o, ac_o, s.lam)
        E_o = 0.5 * float(go @ cho_solve(cho_factor(Vo, lower=True), go))
        del Vo
        print(f"[{tag}] E_J {E:.15e} vs the oracle's 1/2 gamma_o . (V_o + lam I)^-1 gamma_o "
              f"{E_o:.15e} rel {abs(E - E_o) / abs(E_o):.2e}", flush=True)
        assert abs(E - E_o) < REL_E * abs(E_o)
    else:
        # (b) adjoint identity between the forward and reverse kernels
        v = torch.tensor(rng.normal(size=N), device="cuda")
        Jv = _ri._gamma_vjp(x, v, None)[0]
        q = _scr.density_pairs(C, s.occ, pi, pj) * w
        lhs = float(torch.dot(v, gam))
        terms = q * Jv
        rhs = float(terms.sum())
        scale = float(terms.abs().sum())
        print(f"[{tag}] v.gamma {lhs:.15e} vs sum_a q_a J_a(v) {rhs:.15e}: "
              f"diff / sum|terms| {abs(lhs - rhs) / scale:.2e}", flush=True)
        assert abs(lhs - rhs) < 1e-12 * scale
        # (c) normwise backward error of the solve against the metric built afresh
        r = torch.mv(V, d) - gam
        eta = float(r.abs().max()) / (float(V.abs().sum(1).max()) * float(d.abs().max())
                                     + float(gam.abs().max()))
        print(f"[{tag}] solve backward error {eta:.2e}; E_J {E:.15e}", flush=True)
        assert eta < 1e-12
    del V
    torch.cuda.empty_cache()


# ----------------------------------------------------------------------------- launch geometry

def test_forward_grid_past_one_grid_dimension(g, wl, cuda):
    """The forward's workgroups (pair groups x aux record blocks) outnumber what one grid dimension
    holds (2^32 - 1 work-items) on the 700-atom globule's list grown to 1.86 n0 (eps 5e-12:
    20.7 M pairs against 80000 aux functions, as a trainer's pad allows). gamma is linear in the
    list, so gamma of the whole list must equal gamma of its two halves added (each half within
    one grid dimension even as a one-dimensional grid), to the round-off of the regrouped sums."""
    from gs_dft_amd import ri as _ri
    eps = 5e-12
    s = wl.make_system(5, eps=eps)
    basis = _splat(g, s)
    pi, pj, w = g.neighbor_pairs(basis, eps, unique=True)
    aux = g.init_product_aux(basis, scales=s.scales)
    C = torch.tensor(s.C, device="cuda")
    x = _ri._Inputs(basis, C, s.occ, aux, pi, pj, w, None)
    n, N = x.n_live, aux.n_basis
    groups, rec_blocks = (n + 8191) // 8192, (N + 11) // 12
    print(f"[grid] n={n} N_aux={N}: {groups} pair groups x {rec_blocks} record blocks x 256 = "
          f"{groups * rec_blocks * 256:.3e} work-items", flush=True)
    assert groups * rec_blocks * 256 > 2 ** 32
    gam = _ri._gamma_forward(x)
    h = n // 2
    halves = [_ri._Inputs(basis, C, s.occ, aux, pi[a:b], pj[a:b], w[a:b], None)
              for a, b in ((0, h), (h, n))]
    assert all(((hx.n_live + 8191) // 8192) * rec_blocks * 256 < 2 ** 32 for hx in halves)
    gsum = _ri._gamma_forward(halves[0]) + _ri._gamma_forward(halves[1])
    torch.cuda.synchronize()
    err = float(((gam - gsum).abs() / gam.abs()).max())
    print(f"[grid] gamma of the whole list vs its halves added: max elementwise rel {err:.2e}",
          flush=True)
    assert err < 1e-12
    del gam, gsum, x, halves
    torch.cuda.empty_cache()
