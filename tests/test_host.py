"""Host-side plugin surface (no GPU): spec values, validation and errors mirror
gs_dft/ks/terms.py and gs_dft/ks/train.py."""
import pytest


def test_df_spec_defaults_and_validation(g):
    d = g.df()
    assert d == g.DFSpec(scales=(1.0,), diagonal=True, lam=1e-8, chunk=2048)
    assert g.df(scales=(0.5, 1, 2)).scales == (0.5, 1.0, 2.0)
    with pytest.raises(ValueError, match="at least one"):
        g.df(scales=())


def test_pairlist_defaults(g):
    p = g.pairlist()
    assert (p.eps, p.pad, p.unique, p.skip_pad) == (1e-7, g.SCREEN_PAD, False, False)
    assert g.SCREEN_PAD == 2.0
    assert g.pairlist(1e-5, unique=True).unique is True


def test_make_coulomb_resolves_the_screened_strategies(g):
    """gs_dft/ks/terms.py:273-301: df() and exact() with a screen resolve to their screened terms
    (exact() with the reference's default chunk 128), exact() without one to
    StreamedExactCoulomb (default chunk 64), df() with a hybrid carries its a_x and a
    range-separated one its a_x_lr and omega; dense DF and hybrids on the exact paths raise."""
    from gs_dft_amd.terms import _make_coulomb
    t = _make_coulomb(g.df(lam=1e-6), screened=True, skip_pad=True)
    assert isinstance(t, g.ScreenedProductDFCoulomb) and t.lam == 1e-6 and t.skip_pad
    e = _make_coulomb(g.exact(), screened=True)
    assert isinstance(e, g.ScreenedExactCoulomb) and e.chunk == 128 and e.hf_coeff == 0.0
    assert _make_coulomb(g.exact(chunk=32), screened=True).chunk == 32
    with pytest.raises(NotImplementedError):
        _make_coulomb(g.df(), screened=False)
    st = _make_coulomb(g.exact(), screened=False)
    assert isinstance(st, g.StreamedExactCoulomb) and st.chunk == 64 and st.hf_coeff == 0.0
    assert _make_coulomb(g.exact(chunk=16), screened=False).chunk == 16
    with pytest.raises(NotImplementedError, match="M\\^4 ERI tensor"):
        _make_coulomb(g.exact(), screened=False, a_x=0.25)
    with pytest.raises(ValueError):
        _make_coulomb(g.exact(), screened=False, a_x_lr=0.5)
    assert isinstance(g.SplatDFJ(coulomb=g.exact()).coulomb, g.StreamedExactCoulomb)
    with pytest.raises(NotImplementedError):
        g.SplatDFJ(coulomb=g.df())
    with pytest.raises(ValueError):
        _make_coulomb(g.exact(), screened=True, a_x=0.25)
    with pytest.raises(ValueError):
        _make_coulomb(g.exact(), screened=True, a_x_lr=0.5)
    hyb = _make_coulomb(g.df(), screened=True, a_x=0.25)
    assert isinstance(hyb, g.ScreenedProductDFCoulomb) and hyb.hf_coeff == 0.25
    rsh = _make_coulomb(g.df(), screened=True, a_x=0.25, a_x_lr=0.5, omega=0.3)
    assert (rsh.hf_coeff, rsh.hf_coeff_lr, rsh.omega) == (0.25, 0.5, 0.3)
    with pytest.raises(TypeError):
        _make_coulomb("df", screened=True)


def test_hybrid_checks_mirror_the_reference(g):
    """gs_dft/ks/energy.py:240-241 (unique lists are PBE-class only), 283-285 (hybrid df() needs
    state.aux_K, here also for a purely long-range xc); a negative or infinite omega is refused
    before any device work."""

    class Hybrid:
        exact_exchange_fraction = 0.25

    with pytest.raises(ValueError, match="unique=True"):
        g.SplatDFJ(coulomb=g.df(), screen=g.pairlist(unique=True), xc=Hybrid())
    ks = g.SplatDFJ(coulomb=g.df(), screen=g.pairlist(), xc=Hybrid())
    assert ks.coulomb.hf_coeff == 0.25 and g.hf_coeff(Hybrid()) == 0.25
    with pytest.raises(ValueError, match="aux_K"):
        ks._check_state(g.SplatState(pairs=(1, 2, 3), aux=object()))

    class LongRange:
        hf_coeff_lr = 1.0
        omega = 0.4

    lr = g.SplatDFJ(coulomb=g.df(), screen=g.pairlist(), xc=LongRange())
    assert (lr.coulomb.hf_coeff, lr.coulomb.hf_coeff_lr, lr.coulomb.omega) == (0.0, 1.0, 0.4)
    with pytest.raises(ValueError, match="aux_K"):
        lr._check_state(g.SplatState(pairs=(1, 2, 3), aux=object()))
    for bad in (-0.3, float("inf"), float("nan")):
        with pytest.raises(ValueError, match="omega"):
            g.df_exchange_energy_screened(None, None, None, None, None, omega=bad)


def test_train_pad_rule(g):
    """pad_to = ceil(pad * n0 / G) * G (gs_dft/ks/train.py:359)."""
    assert g.train_pad_to(g.pairlist(), 1001) == 2002
    assert g.train_pad_to(g.pairlist(pad=1.5), 1001, 4) == 1504
    assert g.train_pad_to(g.pairlist(pad=1.25), 7) == 8


def test_state_checks(g):
    ks = g.SplatDFJ(coulomb=g.df(), screen=g.pairlist())
    with pytest.raises(ValueError, match="state.pairs"):
        ks._check_state(g.SplatState())
    with pytest.raises(ValueError, match="product aux"):
        ks._check_state(g.SplatState(pairs=(1, 2, 3)))
    with pytest.raises(NotImplementedError):
        g.SplatDFJ(coulomb=g.df(), screen=None)
    with pytest.raises(NotImplementedError):
        g.SplatDFJ(coulomb=g.df(), screen=g.pairlist(), mesh=object())


def test_workloads_are_deterministic_and_sized(wl):
    a, b = wl.make_system(1), wl.make_system(1)
    assert (a.quat == b.quat).all() and (a.C == b.C).all()
    assert (a.M, a.k, a.n_aux) == (126, 11, 504)
    s3 = wl.make_system(3)
    assert (s3.M, s3.k, s3.n_aux) == (2000, 81, 8000) and s3.atoms.shape == (62, 3)
    import numpy as np
    assert abs(np.linalg.norm(s3.C, axis=0).mean() - np.sqrt(2000 / 81)) < 0.5


def test_pair_index_range_check(g):
    """The host check every pair-list entry point runs before a launch: indices outside
    [0, bound) raise ValueError, since the kernels read the rows they name unchecked."""
    import torch
    from gs_dft_amd.screening import check_pair_indices
    ok = torch.tensor([0, 3, 4], dtype=torch.int32)
    check_pair_indices(ok, ok.flip(0), 5, "t")
    check_pair_indices(ok[:0], ok[:0], 5, "t")
    with pytest.raises(ValueError, match=r"\[0, 5\)"):
        check_pair_indices(ok, torch.tensor([0, 5, 1], dtype=torch.int32), 5, "t")
    with pytest.raises(ValueError, match=r"got \[-1, 4\]"):
        check_pair_indices(torch.tensor([-1, 0, 4], dtype=torch.int32), ok, 5, "t")
    with pytest.raises(ValueError, match="same length"):
        check_pair_indices(ok, ok[:2], 5, "t")


def test_exchange_symmetry_check_compares_weights(g):
    """The RI-K symmetric path drops the antisymmetric part of every D_P, which is exact only when
    the live entries come in (i, j) / (j, i) pairs of equal weight: a list with the same pattern
    but a different weight on one order, or an entry whose mirror is dead, takes the general path;
    repeats count as a multiset."""
    import torch
    from gs_dft_amd.ri import _list_symmetric
    pi = torch.tensor([0, 1, 2, 0, 3], dtype=torch.int32)
    pj = torch.tensor([1, 0, 2, 3, 0], dtype=torch.int32)
    w = torch.tensor([1.0, 1.0, 1.0, 0.5, 0.5], dtype=torch.float64)
    assert _list_symmetric(4, pi, pj, w, 5)
    assert not _list_symmetric(4, pi, pj, torch.tensor([1.0, 2.0, 1.0, 0.5, 0.5]), 5)
    assert not _list_symmetric(4, pi, pj, torch.tensor([1.0, 1.0, 1.0, 0.5, 0.0]), 5)
    assert _list_symmetric(4, pi, pj, torch.tensor([1.0, 1.0, 1.0, 0.0, 0.0]), 5)
    pr = torch.tensor([0, 0, 1, 1], dtype=torch.int32)
    pc = torch.tensor([1, 1, 0, 0], dtype=torch.int32)
    assert _list_symmetric(2, pr, pc, torch.tensor([1.0, 2.0, 2.0, 1.0]), 4)
    assert not _list_symmetric(2, pr, pc, torch.tensor([1.0, 2.0, 2.0, 2.0]), 4)
    assert _list_symmetric(4, pi, pj, w, 0)
