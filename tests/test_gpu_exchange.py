"""Parity of the HIP screened RI-K exchange (gs_dft/coulomb/ri.py:497-544) against the CPU oracle
(E_K) and autograd of the torch literal restatement (gradients), on the same seeded inputs; at
the water octamer's full size through size-independent identities.

Bars: E_K within 1e-10 relative; gradients w.r.t. the splat leaves and C within 1e-9 relative to
the largest entry.
"""
import numpy as np
import pytest
import torch

from conftest import rel_max

pytestmark = pytest.mark.gpu

REL_E = 1e-10
REL_G = 1e-9


def _cu(a, grad=False):
    return torch.tensor(np.asarray(a), device="cuda", dtype=torch.float64).requires_grad_(grad)


def _t(x, grad=False):
    t = torch.as_tensor(np.asarray(x), dtype=torch.float64).clone()
    return t.requires_grad_(grad) if grad else t


def _idx(a):
    return torch.as_tensor(np.asarray(a, dtype=np.int64))


def _np(t):
    return t.detach().cpu().numpy()


def _basis(g, s, grad=True):
    return g.Splat(quat=_cu(s.quat, grad), log_scale=_cu(s.log_scale, grad),
                   centers=_cu(s.centers, grad))


@pytest.mark.parametrize("masked", [False, True])
@pytest.mark.parametrize("k,aux_chunk,recompute", [(1, 0, False), (4, 37, False), (4, 37, True),
                                                   (7, 0, True), (33, 0, False),
                                                   (130, 0, True)])
def test_exchange_matches_oracle_and_autograd(g, wl, orc, tr, cuda, masked, k, aux_chunk,
                                              recompute):
    s = wl.make_small(30, k, n_atoms=3, seed=5 + k)
    la, ac = orc.product_aux(s.quat, s.log_scale, s.centers, s.scales)
    pi, pj, w, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, 1e-7, None, False)
    w = w.astype(np.float64)
    if masked:                      # drops entries one-sidedly: the list is no longer symmetric
        w = w * (np.random.default_rng(k).uniform(size=w.shape) > 0.15)
    print(f"[exchange] M={s.M} k={k} N={len(la)} n={len(pi)} masked={masked} "
          f"aux_chunk={aux_chunk} recompute={recompute}", flush=True)
    basis, C = _basis(g, s), _cu(s.C, True)
    aux = g.IsotropicSplat(log_alpha=la, centers=ac)
    E = g.df_exchange_energy_screened(basis, C, aux, torch.tensor(pi, device="cuda"),
                                      torch.tensor(pj, device="cuda"), lam=1e-8,
                                      valid=torch.tensor(w, device="cuda"), aux_chunk=aux_chunk,
                                      recompute=recompute)
    Eo, _ = orc.exchange_energy(s.quat, s.log_scale, s.centers, s.C, la, ac, pi, pj, w, 1e-8)
    err = abs(E.item() - Eo) / abs(Eo)
    print(f"[exchange] E_K {E.item():.15e} oracle {Eo:.15e} rel {err:.2e}")
    assert err < REL_E
    E.backward()
    leaves = [_t(s.quat, True), _t(s.log_scale, True), _t(s.centers, True), _t(s.C, True)]
    Et = tr.screened_exchange_energy(*leaves, _t(la), _t(ac), _idx(pi), _idx(pj), _t(w), 1e-8)
    Et.backward()
    for name, a, b in zip(("quat", "log_scale", "centers", "C"),
                          (basis.quat, basis.log_scale, basis.centers, C), leaves):
        e = rel_max(_np(a.grad), b.grad.numpy())
        print(f"[exchange] d{name} rel-to-max {e:.2e}")
        assert e < REL_G


@pytest.mark.parametrize("aux_chunk", [0, 37])
def test_exchange_repeated_entries(g, wl, orc, tr, cuda, aux_chunk):
    """Entries the three-centre passes share: a list whose entries repeat (some (i, k) twice, with
    and without their (k, i)), a self pair repeated, and dead entries (weight 0) among the live
    ones -- groups of one, two, three and four entries of one unordered splat pair, against the
    oracle's and the torch literal's entry-by-entry contraction."""
    k = 5
    s = wl.make_small(30, k, n_atoms=3, seed=11)
    la, ac = orc.product_aux(s.quat, s.log_scale, s.centers, s.scales)
    pi, pj, w, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, 1e-7, None, False)
    w = w.astype(np.float64)
    rng = np.random.default_rng(4)
    off = np.flatnonzero(pi != pj)
    rep = rng.choice(off, size=len(off) // 5, replace=False)      # (i, k) again
    selfp = np.flatnonzero(pi == pj)[:3]                           # (i, i) again
    mirror = rep[: len(rep) // 2]                                  # and some (k, i) again
    pi2 = np.concatenate([pi, pi[rep], pi[selfp], pj[mirror]]).astype(np.int32)
    pj2 = np.concatenate([pj, pj[rep], pj[selfp], pi[mirror]]).astype(np.int32)
    w2 = np.concatenate([w, w[rep], w[selfp], w[mirror]])
    dead = rng.choice(len(w2), size=len(w2) // 10, replace=False)
    w2[dead] = 0.0
    print(f"[exchange] repeated entries: n={len(pi2)} (list {len(pi)}, +{len(rep)} repeats, "
          f"+{len(selfp)} self, +{len(mirror)} mirrors, {len(dead)} dead) aux_chunk={aux_chunk}",
          flush=True)
    basis, C = _basis(g, s), _cu(s.C, True)
    aux = g.IsotropicSplat(log_alpha=la, centers=ac)
    E = g.df_exchange_energy_screened(basis, C, aux, torch.tensor(pi2, device="cuda"),
                                      torch.tensor(pj2, device="cuda"), lam=1e-8,
                                      valid=torch.tensor(w2, device="cuda"), aux_chunk=aux_chunk)
    Eo, _ = orc.exchange_energy(s.quat, s.log_scale, s.centers, s.C, la, ac, pi2, pj2, w2, 1e-8)
    err = abs(E.item() - Eo) / abs(Eo)
    print(f"[exchange] E_K {E.item():.15e} oracle {Eo:.15e} rel {err:.2e}")
    assert err < REL_E
    E.backward()
    leaves = [_t(s.quat, True), _t(s.log_scale, True), _t(s.centers, True), _t(s.C, True)]
    Et = tr.screened_exchange_energy(*leaves, _t(la), _t(ac), _idx(pi2), _idx(pj2), _t(w2), 1e-8)
    Et.backward()
    for name, a, b in zip(("quat", "log_scale", "centers", "C"),
                          (basis.quat, basis.log_scale, basis.centers, C), leaves):
        e = rel_max(_np(a.grad), b.grad.numpy())
        print(f"[exchange] d{name} rel-to-max {e:.2e}")
        assert e < REL_G


@pytest.mark.parametrize("aux_chunk", [0, 37])
def test_exchange_symmetric_list_with_dead_pairs(g, wl, orc, tr, cuda, aux_chunk):
    """A list that stays symmetric with some pairs dead in both orders (weight 0 for (i, k) and
    (k, i)): the symmetric path, whose sampled product forms rows for the live groups only --
    E_K and gradients against the oracle and the torch literal."""
    from gs_dft_amd import ri
    k = 4
    s = wl.make_small(30, k, n_atoms=3, seed=17)
    la, ac = orc.product_aux(s.quat, s.log_scale, s.centers, s.scales)
    pi, pj, w, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, 1e-7, None, False)
    w = w.astype(np.float64)
    rng = np.random.default_rng(8)
    lo, hi = np.minimum(pi, pj), np.maximum(pi, pj)
    kill = rng.uniform(size=(s.M, s.M)) < 0.2                      # per unordered pair
    w[kill[lo, hi] & (pi != pj)] = 0.0
    assert ri._list_symmetric(s.M, torch.as_tensor(pi), torch.as_tensor(pj), torch.as_tensor(w),
                              len(pi))
    print(f"[exchange] symmetric with dead pairs: n={len(pi)} dead={int((w == 0).sum())} "
          f"aux_chunk={aux_chunk}", flush=True)
    basis, C = _basis(g, s), _cu(s.C, True)
    aux = g.IsotropicSplat(log_alpha=la, centers=ac)
    E = g.df_exchange_energy_screened(basis, C, aux, torch.tensor(pi, device="cuda"),
                                      torch.tensor(pj, device="cuda"), lam=1e-8,
                                      valid=torch.tensor(w, device="cuda"), aux_chunk=aux_chunk)
    Eo, _ = orc.exchange_energy(s.quat, s.log_scale, s.centers, s.C, la, ac, pi, pj, w, 1e-8)
    err = abs(E.item() - Eo) / abs(Eo)
    print(f"[exchange] E_K {E.item():.15e} oracle {Eo:.15e} rel {err:.2e}")
    assert err < REL_E
    E.backward()
    leaves = [_t(s.quat, True), _t(s.log_scale, True), _t(s.centers, True), _t(s.C, True)]
    Et = tr.screened_exchange_energy(*leaves, _t(la), _t(ac), _idx(pi), _idx(pj), _t(w), 1e-8)
    Et.backward()
    for name, a, b in zip(("quat", "log_scale", "centers", "C"),
                          (basis.quat, basis.log_scale, basis.centers, C), leaves):
        e = rel_max(_np(a.grad), b.grad.numpy())
        print(f"[exchange] d{name} rel-to-max {e:.2e}")
        assert e < REL_G


@pytest.mark.parametrize("aux_chunk", [0, 37])
def test_exchange_integer_weights_through_the_library_call(g, wl, orc, tr, cuda, aux_chunk):
    """gsdft_exchange with weights other than 0/1. The Python entry point, like the reference
    (ri.py:509-520 reads valid as a mask), takes only 0/1; the C interface multiplies each entry by
    its weight, and an entry of integer weight w equals the same entry listed w times. Weights of
    1, 2 or 3 drawn independently for (i, k) and (k, i), plus repeats with other weights: the
    entries of an unordered pair then need three-centre rows of their own (groups split by
    weight) and the list is not symmetric (D_P has an antisymmetric part). E_K and gradients of
    the library call against the oracle and the torch literal on the list with each entry
    repeated w times."""
    from gs_dft_amd import ri
    k = 4
    s = wl.make_small(30, k, n_atoms=3, seed=13)
    la, ac = orc.product_aux(s.quat, s.log_scale, s.centers, s.scales)
    pi, pj, w, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, 1e-7, None, False)
    live = np.flatnonzero(w != 0)
    pi, pj = pi[live], pj[live]
    rng = np.random.default_rng(6)
    rep = rng.choice(len(pi), size=len(pi) // 6, replace=False)    # repeats
    pi2 = np.concatenate([pi, pi[rep]]).astype(np.int32)
    pj2 = np.concatenate([pj, pj[rep]]).astype(np.int32)
    w2 = rng.integers(1, 4, size=len(pi2)).astype(np.float64)
    pie, pje = np.repeat(pi2, w2.astype(int)), np.repeat(pj2, w2.astype(int))
    we = np.ones(len(pie))
    print(f"[exchange] integer weights: n={len(pi2)} (+{len(rep)} repeats), expanded "
          f"{len(pie)}, aux_chunk={aux_chunk}", flush=True)
    basis, C = _basis(g, s, grad=False), _cu(s.C)
    aux = g.IsotropicSplat(log_alpha=la, centers=ac)
    pit, pjt = torch.tensor(pi2, device="cuda"), torch.tensor(pj2, device="cuda")
    x = ri._ExchangeInputs(basis, C, aux, pit, pjt, torch.ones(len(pi2), device="cuda"),
                           ri.aux_cholesky(aux, 1e-8), None, aux_chunk, False)
    x.w = torch.tensor(w2, device="cuda")
    x.symmetric = ri._list_symmetric(x.M, x.pi, x.pj, x.w, x.n)
    assert not x.symmetric and x.n == len(pi2)
    E, dq, dl, dc, dC = ri._exchange(x, True)
    Eo, _ = orc.exchange_energy(s.quat, s.log_scale, s.centers, s.C, la, ac, pie, pje, we, 1e-8)
    err = abs(E.item() - Eo) / abs(Eo)
    print(f"[exchange] E_K {E.item():.15e} oracle {Eo:.15e} rel {err:.2e}")
    assert err < REL_E
    leaves = [_t(s.quat, True), _t(s.log_scale, True), _t(s.centers, True), _t(s.C, True)]
    Et = tr.screened_exchange_energy(*leaves, _t(la), _t(ac), _idx(pie), _idx(pje), _t(we), 1e-8)
    Et.backward()
    for name, a, b in zip(("quat", "log_scale", "centers", "C"), (dq, dl, dc, dC), leaves):
        e = rel_max(_np(a), b.grad.numpy())
        print(f"[exchange] d{name} rel-to-max {e:.2e}")
        assert e < REL_G


@pytest.mark.parametrize("case", ["one_self_pair", "self_pairs_only", "one_pair_both_ways"])
def test_exchange_tiny_lists(g, wl, orc, tr, cuda, case):
    """Lists of one or a few groups: a single self pair, self pairs only, and one off-diagonal
    pair listed both ways (a single group of two entries) -- E_K and gradients against the
    oracle and the torch literal."""
    k = 3
    s = wl.make_small(12, k, n_atoms=2, seed=21)
    la, ac = orc.product_aux(s.quat, s.log_scale, s.centers, s.scales)
    if case == "one_self_pair":
        pi, pj = np.array([4]), np.array([4])
    elif case == "self_pairs_only":
        pi = pj = np.arange(s.M)
    else:
        pi, pj = np.array([2, 7]), np.array([7, 2])
    pi, pj = pi.astype(np.int32), pj.astype(np.int32)
    w = np.ones(len(pi))
    basis, C = _basis(g, s), _cu(s.C, True)
    aux = g.IsotropicSplat(log_alpha=la, centers=ac)
    E = g.df_exchange_energy_screened(basis, C, aux, torch.tensor(pi, device="cuda"),
                                      torch.tensor(pj, device="cuda"), lam=1e-8,
                                      valid=torch.tensor(w, device="cuda"))
    Eo, _ = orc.exchange_energy(s.quat, s.log_scale, s.centers, s.C, la, ac, pi, pj, w, 1e-8)
    err = abs(E.item() - Eo) / abs(Eo)
    print(f"[exchange] {case}: n={len(pi)} E_K {E.item():.15e} oracle {Eo:.15e} rel {err:.2e}")
    assert err < REL_E
    E.backward()
    leaves = [_t(s.quat, True), _t(s.log_scale, True), _t(s.centers, True), _t(s.C, True)]
    Et = tr.screened_exchange_energy(*leaves, _t(la), _t(ac), _idx(pi), _idx(pj), _t(w), 1e-8)
    Et.backward()
    for name, a, b in zip(("quat", "log_scale", "centers", "C"),
                          (basis.quat, basis.log_scale, basis.centers, C), leaves):
        e = rel_max(_np(a.grad), b.grad.numpy())
        print(f"[exchange] {case}: d{name} rel-to-max {e:.2e}")
        assert e < REL_G


def _lr_tolerance(cond):
    """Relative bound on E_K[erf(omega r)/r] between two correct evaluations: the erf metric is
    ill-conditioned (cond(V + lam I) ~ 1e9 at lam = 1e-8), and E_K inherits ~cond x eps from
    round-off in V and M (the oracle and the torch literal differ by 1.6e-17 to 8.6e-17 x cond)."""
    return max(1e-12, 1e-15 * cond)


def test_long_range_metric_matches_oracle(g, wl, orc, cuda):
    """The erf(omega r)/r metric (gs_dft/coulomb/ri.py:70-72) on the water octamer's product aux
    against the oracle; omega < 0 is refused."""
    s = wl.make_system(2)
    aux = g.init_product_aux(_basis(g, s, grad=False), scales=s.scales)
    la, ac = orc.product_aux(s.quat, s.log_scale, s.centers, s.scales)
    for om in (0.11, 0.3):
        V = _np(g.aux_metric(aux, om, lam=1e-8))
        Vo = orc.aux_metric(la, ac, 1e-8, om)
        err = np.max(np.abs(V - Vo) / np.abs(Vo))
        print(f"[exchange] erf metric omega={om} N={len(la)} rel {err:.2e}")
        assert err < 1e-13
        assert np.array_equal(V, V.T)
    with pytest.raises(ValueError, match="omega"):
        g.aux_metric(aux, -0.3)


@pytest.mark.parametrize("om,lam,masked", [(0.3, 1e-2, False), (0.3, 1e-8, True),
                                           (0.11, 1e-2, True), (0.11, 1e-8, False)])
def test_long_range_exchange_matches_oracle_and_autograd(g, wl, orc, tr, cuda, om, lam, masked):
    """E_K[erf(omega r)/r] of range-separated hybrids (ri.py:534-544 with omega; the 12-node rule
    on [0, omega], ri.py:231-235) against the oracle and the gradients against autograd of the
    torch literal under the same rule; the bars scale with cond(V_omega + lam I), which at
    lam = 1e-2 keeps them at the 1e-10 / 1e-9 of the 1/r exchange."""
    k = 4
    s = wl.make_small(30, k, n_atoms=3, seed=31)
    la, ac = orc.product_aux(s.quat, s.log_scale, s.centers, s.scales)
    pi, pj, w, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, 1e-7, None, False)
    w = w.astype(np.float64)
    if masked:
        w = w * (np.random.default_rng(7).uniform(size=w.shape) > 0.15)
    cond = np.linalg.cond(orc.aux_metric(la, ac, lam, om))
    tol_e = _lr_tolerance(cond)
    tol_g = max(REL_G, 1e-14 * cond)
    print(f"[exchange-lr] M={s.M} k={k} N={len(la)} n={len(pi)} omega={om} lam={lam} "
          f"masked={masked} cond {cond:.2e}", flush=True)
    basis, C = _basis(g, s), _cu(s.C, True)
    aux = g.IsotropicSplat(log_alpha=la, centers=ac)
    E = g.df_exchange_energy_screened(basis, C, aux, torch.tensor(pi, device="cuda"),
                                      torch.tensor(pj, device="cuda"), lam=lam,
                                      valid=torch.tensor(w, device="cuda"), omega=om)
    Eo, _ = orc.exchange_energy(s.quat, s.log_scale, s.centers, s.C, la, ac, pi, pj, w, lam,
                                omega=om)
    err = abs(E.item() - Eo) / abs(Eo)
    print(f"[exchange-lr] E_K {E.item():.15e} oracle {Eo:.15e} rel {err:.2e} (bar {tol_e:.1e})")
    assert err < tol_e
    E.backward()
    t, wq = orc.lr_quad_table(om)
    leaves = [_t(s.quat, True), _t(s.log_scale, True), _t(s.centers, True), _t(s.C, True)]
    Et = tr.screened_exchange_energy(*leaves, _t(la), _t(ac), _idx(pi), _idx(pj), _t(w), lam,
                                     table=([float(v) for v in t], [float(v) for v in wq]),
                                     omega=om)
    Et.backward()
    for name, a, b in zip(("quat", "log_scale", "centers", "C"),
                          (basis.quat, basis.log_scale, basis.centers, C), leaves):
        e = rel_max(_np(a.grad), b.grad.numpy())
        print(f"[exchange-lr] d{name} rel-to-max {e:.2e} (bar {tol_g:.1e})")
        assert e < tol_g


def test_long_range_plugin_energy(g, wl, cuda):
    """SplatDFJ with a range-separated xc (hf_coeff, hf_coeff_lr, omega) evaluates
    E_J + a E_K + b E_K[erf(omega r)/r] (gs_dft/ks/terms.py:258-264, gs_dft/ks/energy.py:330,
    406-408); a purely long-range xc (hf_coeff = 0) still gets its K-aux from refresh."""

    class RangeSeparated:
        hf_coeff = 0.19
        hf_coeff_lr = 0.46
        omega = 0.33

    class LongRangeOnly:
        hf_coeff = 0.0
        hf_coeff_lr = 1.0
        omega = 0.4

    s = wl.make_small(40, 5, n_atoms=4, seed=9)
    basis, C = _basis(g, s), _cu(s.C, True)
    occ = torch.tensor(s.occ, device="cuda")
    for xc in (RangeSeparated(), LongRangeOnly()):
        ks = g.SplatDFJ(coulomb=g.df(scales=s.scales), screen=g.pairlist(1e-7), xc=xc)
        state = g.refresh(ks, basis)
        assert state.aux_K is state.aux and state.cholV_lr is not None
        model = g.SplatModel(basis=basis, C=C, occupations=occ)
        E = ks(model, state)
        pi, pj, valid = state.pairs
        with torch.no_grad():
            EJ = g.df_coulomb_energy_screened(basis, C, occ, state.aux, pi, pj, valid=valid,
                                              cholV=state.cholV)
            EK = g.df_exchange_energy_screened(basis, C, state.aux, pi, pj, valid=valid)
            ELR = g.df_exchange_energy_screened(basis, C, state.aux, pi, pj, valid=valid,
                                                omega=xc.omega)
        ref = EJ.item() + xc.hf_coeff * EK.item() + xc.hf_coeff_lr * ELR.item()
        print(f"[exchange-lr] plugin E {E.item():.15e} = E_J {EJ.item():.6e} + "
              f"{xc.hf_coeff} E_K {EK.item():.6e} + {xc.hf_coeff_lr} E_K^lr {ELR.item():.6e}")
        assert abs(E.item() - ref) < 1e-12 * abs(E.item())
        # the refresh's erf factor is the one the call would form itself: same energy bit for bit
        with torch.no_grad():
            ELR_state = ks.coulomb.energy_lr(basis, C, None, occ, state)
        assert ELR_state.item() == ELR.item()
        C.grad = None
        E.backward()
        assert torch.isfinite(C.grad).all() and torch.isfinite(basis.centers.grad).all()


def test_exchange_plugin_hybrid_and_state(g, wl, cuda):
    """SplatDFJ with a hybrid xc evaluates E_J + a_x E_K through refresh's K-aux and factor
    (gs_dft/ks/terms.py:245-256, gs_dft/ks/energy.py:400-410, 454-473)."""

    class Hybrid:
        exact_exchange_fraction = 0.25

    s = wl.make_small(40, 5, n_atoms=4, seed=9)
    basis, C = _basis(g, s), _cu(s.C, True)
    ks = g.SplatDFJ(coulomb=g.df(scales=s.scales), screen=g.pairlist(1e-7), xc=Hybrid())
    state = g.refresh(ks, basis)
    assert state.aux_K is state.aux
    model = g.SplatModel(basis=basis, C=C, occupations=torch.tensor(s.occ, device="cuda"))
    E = ks(model, state)
    pi, pj, valid = state.pairs
    EJ = g.df_coulomb_energy_screened(basis, C, model.occupations, state.aux, pi, pj,
                                      valid=valid, cholV=state.cholV)
    EK = g.df_exchange_energy_screened(basis, C, state.aux, pi, pj, valid=valid, lam=1e-8)
    print(f"[exchange] plugin E {E.item():.15e} = E_J {EJ.item():.6e} + 0.25 E_K {EK.item():.6e}")
    assert abs(E.item() - (EJ.item() + 0.25 * EK.item())) < 1e-12 * abs(E.item())
    E.backward()
    assert torch.isfinite(C.grad).all() and torch.isfinite(basis.centers.grad).all()


def test_exchange_water8_identities(g, wl, cuda):
    """The water octamer (M = 600, k = 40, 2400 aux) at full size: E_K is invariant under an
    orthogonal rotation of the occupied orbitals; with one orbital it equals -2 E_J^DF at
    occupation 1 (the DF-J path, parity-pinned on its own); the gradient's directional derivative
    matches central differences of the energy."""
    s = wl.make_system(2)
    basis, C = _basis(g, s), _cu(s.C, True)
    aux = g.init_product_aux(basis, scales=s.scales)
    L = g.aux_cholesky(aux, 1e-8)
    pi, pj, valid = g.neighbor_pairs(basis, eps=1e-7)
    index = g.build_pair_index(s.M, pi, pj, valid)
    print(f"[exchange] water8 M={s.M} k={s.k} N={aux.n_basis} n={index.n_live}", flush=True)

    def ek(Cm, b=basis, **kw):
        return g.df_exchange_energy_screened(b, Cm, aux, pi, pj, valid=valid, cholV=L,
                                             index=index, **kw)

    E = ek(C)
    U, _ = np.linalg.qr(np.random.default_rng(2).normal(size=(s.k, s.k)))
    with torch.no_grad():
        Er = ek(C @ _cu(U), aux_chunk=512, recompute=True)
    e_rot = abs(Er.item() - E.item()) / abs(E.item())
    C1 = C.detach()[:, :1].contiguous()
    with torch.no_grad():
        E1 = ek(C1)
        EJ1 = g.df_coulomb_energy_screened(basis, C1, torch.ones(1, device="cuda",
                                                                  dtype=torch.float64),
                                           aux, pi, pj, valid=valid, cholV=L, index=index)
    e_one = abs(E1.item() + 2 * EJ1.item()) / abs(E1.item())
    print(f"[exchange] water8 E_K {E.item():.12e}: rotation {e_rot:.2e}, k=1 vs -2 E_J {e_one:.2e}")
    assert e_rot < 1e-11 and e_one < 1e-11
    E.backward()
    leaves = (basis.quat, basis.log_scale, basis.centers, C)
    gen = torch.Generator(device="cpu").manual_seed(3)
    dirs = [torch.randn(t.shape, generator=gen, dtype=torch.float64).cuda() for t in leaves]
    dd = sum((t.grad * d).sum().item() for t, d in zip(leaves, dirs))
    h = 1e-5

    def e_at(sign):
        with torch.no_grad():
            b = g.Splat(quat=basis.quat + sign * h * dirs[0],
                        log_scale=basis.log_scale + sign * h * dirs[1],
                        centers=basis.centers + sign * h * dirs[2])
            return ek(C + sign * h * dirs[3], b=b).item()

    fd = (e_at(1) - e_at(-1)) / (2 * h)
    print(f"[exchange] water8 directional derivative {dd:.10e} vs central difference {fd:.10e}")
    assert abs(fd - dd) < 1e-6 * max(1.0, abs(dd))
    # recomputing the forward's products in the reverse (the memory knob) gives the same bits
    grads = [t.grad.clone() for t in leaves]
    for t in leaves:
        t.grad = None
    ek(C, recompute=True).backward()
    assert all(torch.equal(a, t.grad) for a, t in zip(grads, leaves))
