"""Parity of the HIP exact pair-pair Coulomb (gs_dft/coulomb/stream.py:249-320) against the CPU
oracle (the reference's Schur-complement node form) and autograd of the torch literal
restatement, on the same seeded inputs.

Bars: E_J and J within 1e-10 relative (observed ~1e-14); gradients within 1e-9 relative to the
largest entry.
"""
import numpy as np
import pytest
import torch

from conftest import rel_max

pytestmark = pytest.mark.gpu

REL_E = 1e-10
REL_G = 1e-9

SMALL = [dict(M=24, k=5, n_atoms=3, seed=1), dict(M=40, k=6, n_atoms=4, seed=5, spread=3.0),
         dict(M=200, k=9, n_atoms=8, seed=3, spread=6.0)]


def _small(wl, spec):
    spec = dict(spec)
    return wl.make_small(spec.pop("M"), spec.pop("k"), **spec)


def _cu(a, grad=False):
    return torch.tensor(np.asarray(a), device="cuda", dtype=torch.float64).requires_grad_(grad)


def _np(t):
    return t.detach().cpu().numpy()


def _t(x, grad=False):
    t = torch.as_tensor(np.asarray(x), dtype=torch.float64).clone()
    return t.requires_grad_(grad) if grad else t


def _idx(a):
    return torch.as_tensor(np.asarray(a, dtype=np.int64))


def _gpu(g, s, pi, pj, w):
    basis = g.Splat(quat=_cu(s.quat, True), log_scale=_cu(s.log_scale, True),
                    centers=_cu(s.centers, True))
    C = _cu(s.C, True)
    E = g.screened_coulomb_energy(basis, C, s.occ, pi, pj, valid=w)
    E.backward()
    return (E.item(), _np(basis.quat.grad), _np(basis.log_scale.grad), _np(basis.centers.grad),
            _np(C.grad))


@pytest.mark.parametrize("case", [0, 1])
def test_exact_energy_J_and_gradients_match(g, wl, orc, tr, cuda, case):
    s = _small(wl, SMALL[case])
    pi, pj, w, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, s.eps, None, True)
    print(f"[eri] small{case}: M={s.M} n={len(pi)}", flush=True)
    got = _gpu(g, s, pi, pj, w)
    E_ref, J_ref = orc.exact_coulomb(s.quat, s.log_scale, s.centers, s.C, s.occ, pi, pj, w)
    rel = abs(got[0] - E_ref) / abs(E_ref)
    print(f"[eri] small{case}: E gpu {got[0]:.15e} oracle {E_ref:.15e} rel {rel:.2e}")
    assert rel < REL_E
    basis = g.Splat(quat=_cu(s.quat), log_scale=_cu(s.log_scale), centers=_cu(s.centers))
    J = _np(g.screened_coulomb_J(basis, _cu(s.C), s.occ, pi, pj, valid=w))
    print(f"[eri] small{case}: J rel-to-max {rel_max(J, J_ref):.2e}")
    assert rel_max(J, J_ref) < REL_E
    leaves = [_t(s.quat, True), _t(s.log_scale, True), _t(s.centers, True), _t(s.C, True)]
    Et = tr.screened_coulomb_energy(*leaves, _t(s.occ), _idx(pi), _idx(pj), _t(w))
    Et.backward()
    for name, a, b in zip(("quat", "log_scale", "centers", "C"), got[1:], leaves):
        err = rel_max(a, b.grad.numpy())
        print(f"[eri] small{case}: d{name} rel-to-max {err:.2e}")
        assert err < REL_G


def test_exact_J_sampled_on_a_larger_list(g, wl, orc, cuda):
    """M = 200 (n ~ 1.2e4 pairs): J on a sample of bra pairs against oracle rows of (a|b) Pw."""
    s = _small(wl, SMALL[2])
    pi, pj, w, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, s.eps, None, True)
    basis = g.Splat(quat=_cu(s.quat), log_scale=_cu(s.log_scale), centers=_cu(s.centers))
    J = _np(g.screened_coulomb_J(basis, _cu(s.C), s.occ, pi, pj, valid=w))
    Pw = w * np.sum(s.occ[None, :] * s.C[pi] * s.C[pj], axis=1)
    sel = np.sort(np.random.default_rng(0).choice(len(pi), 48, replace=False))
    rows = orc.eri_block(s.quat, s.log_scale, s.centers, pi[sel], pj[sel], pi, pj)
    Jref = rows @ Pw
    err = float(np.max(np.abs(J[sel] - Jref) / np.abs(Jref)))
    print(f"[eri] small2 n={len(pi)}: sampled J max elementwise rel {err:.2e}")
    assert err < 1e-12


def test_exact_unique_ordered_padding_determinism_and_df_bound(g, wl, orc, cuda):
    s = _small(wl, SMALL[1])
    pu, qu, wu, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, s.eps, None, True)
    po, qo, wo, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, s.eps, None, False)
    pp, qp, wp, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, s.eps, len(pu) + 50, True)
    a = _gpu(g, s, pu, qu, wu)
    b = _gpu(g, s, po, qo, wo)
    c = _gpu(g, s, pp, qp, wp)
    d = _gpu(g, s, pu, qu, wu)
    assert abs(a[0] - b[0]) < 1e-12 * abs(a[0])
    for x, y in zip(a[1:], b[1:]):
        assert rel_max(x, y) < 1e-11
    for x, y in zip(a, c):                      # appended padding changes nothing, bit for bit
        assert np.array_equal(np.asarray(x), np.asarray(y))
    for x, y in zip(a, d):                      # repeated runs are bit-identical
        assert np.array_equal(np.asarray(x), np.asarray(y))
    # gs-dft tests/unit/test_coulomb_df.py:54: robust DF never exceeds the exact energy
    fi, fj, fw, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, -1.0, None, True)
    ex = g.SplatDFJ(coulomb=g.exact(), screen=g.pairlist(-1.0, unique=True))
    df = g.SplatDFJ(coulomb=g.df(scales=(0.5, 1.0, 2.0, 4.0)), screen=g.pairlist(-1.0, unique=True))
    basis = g.Splat(quat=_cu(s.quat), log_scale=_cu(s.log_scale), centers=_cu(s.centers))
    model = g.SplatModel(basis=basis, C=_cu(s.C), occupations=_cu(s.occ))
    e_ex = ex(model, g.refresh(ex, basis)).item()
    e_df = df(model, g.refresh(df, basis)).item()
    E_ref, _ = orc.exact_coulomb(s.quat, s.log_scale, s.centers, s.C, s.occ, fi, fj, fw)
    print(f"[eri] full list: exact {e_ex:.12e} (oracle {E_ref:.12e}), DF {e_df:.12e}")
    assert abs(e_ex - E_ref) < REL_E * abs(E_ref)
    assert e_df <= e_ex * (1 + 1e-9)


def test_exact_empty_list(g, wl, cuda):
    s = _small(wl, SMALL[0])
    z = np.zeros(0, np.int32)
    basis = g.Splat(quat=_cu(s.quat, True), log_scale=_cu(s.log_scale, True),
                    centers=_cu(s.centers, True))
    E = g.screened_coulomb_energy(basis, _cu(s.C), s.occ, z, z, valid=np.zeros(0))
    E.backward()
    assert E.item() == 0.0 and float(basis.centers.grad.abs().max()) == 0.0


def test_exact_water8_directional_derivative(g, wl, orc, cuda):
    """(H2O)8 (M = 600, ~1.7e5 pairs, ~2.8e10 pair-pairs): the gradient's directional derivative
    against central differences of the GPU energy, through the plugin surface."""
    s = wl.make_system(2)
    ks = g.SplatDFJ(coulomb=g.exact(), screen=g.pairlist(s.eps, unique=True))
    basis = g.Splat(quat=_cu(s.quat, True), log_scale=_cu(s.log_scale, True),
                    centers=_cu(s.centers, True))
    state = g.refresh(ks, basis)
    C = _cu(s.C, True)
    occ = _cu(s.occ)
    E = ks(g.SplatModel(basis=basis, C=C, occupations=occ), state)
    E.backward()
    leaves = (basis.quat, basis.log_scale, basis.centers, C)
    gen = torch.Generator(device="cpu").manual_seed(4)
    dirs = [torch.randn(t.shape, generator=gen, dtype=torch.float64).cuda() for t in leaves]
    dd = sum((t.grad * d).sum().item() for t, d in zip(leaves, dirs))
    h = 1e-5

    def e_at(sign):
        with torch.no_grad():
            b = g.Splat(quat=basis.quat + sign * h * dirs[0],
                        log_scale=basis.log_scale + sign * h * dirs[1],
                        centers=basis.centers + sign * h * dirs[2])
            return ks(g.SplatModel(basis=b, C=C + sign * h * dirs[3], occupations=occ),
                      state).item()

    fd = (e_at(1) - e_at(-1)) / (2 * h)
    print(f"[eri] water8 E {E.item():.10e}: directional derivative {dd:.10e} vs central "
          f"difference {fd:.10e}")
    assert abs(fd - dd) < 1e-6 * max(1.0, abs(dd))


def test_exact_water8_energy_paths_and_sampled_J(g, wl, orc, cuda):
    """(H2O)8 at full size, where the energy-only pass runs in several bands of bra pairs and
    evaluates each unordered pair-pair once: its E_J equals the reverse pass's (which evaluates
    every ordered pair-pair) to round-off, and its J on sampled pairs matches oracle rows of
    (a|b) Pw over the whole list."""
    s = wl.make_system(2)
    pi, pj, w, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, s.eps, None, True)
    print(f"[eri] water8 n={len(pi)}", flush=True)
    basis = g.Splat(quat=_cu(s.quat, True), log_scale=_cu(s.log_scale, True),
                    centers=_cu(s.centers, True))
    C = _cu(s.C, True)
    E_rev = g.screened_coulomb_energy(basis, C, s.occ, pi, pj, valid=w)
    E_rev.backward()
    with torch.no_grad():
        E_fwd = g.screened_coulomb_energy(basis, C, s.occ, pi, pj, valid=w)
        J = _np(g.screened_coulomb_J(basis, C, s.occ, pi, pj, valid=w))
    rel = abs(E_fwd.item() - E_rev.item()) / abs(E_rev.item())
    print(f"[eri] water8 E energy-only {E_fwd.item():.15e} reverse {E_rev.item():.15e} rel {rel:.2e}")
    assert rel < 1e-12
    Pw = w * np.sum(s.occ[None, :] * s.C[pi] * s.C[pj], axis=1)
    rng = np.random.default_rng(7)
    sel = np.sort(np.concatenate([rng.choice(len(pi), 24, replace=False),
                                  [0, len(pi) - 1, 16383, 16384, 40000]]))
    rows = orc.eri_block(s.quat, s.log_scale, s.centers, pi[sel], pj[sel], pi, pj)
    Jref = rows @ Pw
    err = float(np.max(np.abs(J[sel] - Jref) / np.abs(Jref)))
    print(f"[eri] water8 sampled J max elementwise rel {err:.2e}")
    assert err < 1e-12


@pytest.mark.parametrize("unique", [True, False])
def test_full_coulomb_energy_with_a_general_density_matrix(g, wl, orc, tr, cuda, unique):
    """full_coulomb_energy(splats, P) (gs_dft/coulomb/stream.py:284-287) over every basis pair
    (make_pairs, stream.py:47-60) with a density matrix that is not C occ C^T: a random indefinite
    symmetric P on the unique list, a random non-symmetric one on the ordered list. E_J and the
    Coulomb matrix against the oracle's Schur-form block; the splat gradients against autograd of
    the torch literal form; dE/dP against the reference's custom VJP, the Coulomb matrix J with
    the symmetric fill on the unique list (stream.py:127-134,159-167), which on the unique list is
    the symmetrised autograd gradient (G + G^T) / 2."""
    s = _small(wl, SMALL[0])
    M = s.M
    rng = np.random.default_rng(11 + int(unique))
    X = rng.normal(size=(M, M))
    P = 0.5 * (X + X.T) if unique else X
    if unique:
        pi, pj = np.triu_indices(M)
        w = np.where(pi == pj, 1.0, 2.0)
    else:
        pi, pj = np.repeat(np.arange(M), M), np.tile(np.arange(M), M)
        w = np.ones(M * M)
    print(f"[full-eri] M={M} unique={unique} n={len(pi)}", flush=True)
    B = orc.eri_block(s.quat, s.log_scale, s.centers, pi, pj, pi, pj)
    Pw = w * P[pi, pj]
    Jv = B @ Pw
    E_ref = 0.5 * float(Pw @ Jv)
    Jm_ref = np.zeros((M, M))
    Jm_ref[pi, pj] = Jv
    if unique:
        Jm_ref[pj, pi] = Jv
    basis = g.Splat(quat=_cu(s.quat, True), log_scale=_cu(s.log_scale, True),
                    centers=_cu(s.centers, True))
    Pd = _cu(P, True)
    E = g.full_coulomb_energy(basis, Pd, unique=unique)
    E.backward()
    rel = abs(E.item() - E_ref) / abs(E_ref)
    print(f"[full-eri] E gpu {E.item():.15e} oracle {E_ref:.15e} rel {rel:.2e}", flush=True)
    assert rel < REL_E
    errP = rel_max(_np(Pd.grad), Jm_ref)
    Jm = _np(g.full_coulomb_J(basis, Pd.detach(), unique=unique))
    errJ = rel_max(Jm, Jm_ref)
    print(f"[full-eri] dE/dP rel-to-max {errP:.2e}, full_coulomb_J {errJ:.2e}", flush=True)
    assert errP < REL_E and errJ < REL_E
    assert rel_max(Jm, _np(Pd.grad)) < 1e-13     # the forward and reverse kernels' J
    leaves = [_t(s.quat, True), _t(s.log_scale, True), _t(s.centers, True), _t(P, True)]
    Et = tr.full_coulomb_energy(*leaves, unique=unique)
    Et.backward()
    for name, a, b in zip(("quat", "log_scale", "centers"),
                          (basis.quat.grad, basis.log_scale.grad, basis.centers.grad), leaves):
        err = rel_max(_np(a), b.grad.numpy())
        print(f"[full-eri] d{name} rel-to-max {err:.2e}", flush=True)
        assert err < REL_G
    Gt = leaves[3].grad.numpy()
    if unique:
        Gt = 0.5 * (Gt + Gt.T)
    assert rel_max(_np(Pd.grad), Gt) < REL_G


def test_streamed_exact_term_equals_the_screened_full_list(g, wl, cuda):
    """coulomb=exact() without a screen resolves to StreamedExactCoulomb (gs_dft/ks/terms.py:
    180-191,299-300) and reads P = C diag(occ) C^T (gs_dft/ks/energy.py:335); with every pair kept
    (eps < 0) the screened exact term computes the same energy from the same C (the reference's
    full-list-equals-dense relation, tests/unit/test_coulomb_df.py:107), and the gradients with
    respect to C agree. A hybrid functional on the streamed path is refused."""
    s = wl.make_system(1)
    mk = lambda a: _cu(a, True)
    b1 = g.Splat(quat=mk(s.quat), log_scale=mk(s.log_scale), centers=mk(s.centers))
    b2 = g.Splat(quat=mk(s.quat), log_scale=mk(s.log_scale), centers=mk(s.centers))
    C1, C2 = mk(s.C), mk(s.C)
    occ = _cu(s.occ)
    ks1 = g.SplatDFJ(coulomb=g.exact())
    assert isinstance(ks1.coulomb, g.StreamedExactCoulomb)
    E1 = ks1(g.SplatModel(basis=b1, C=C1, occupations=occ), g.refresh(ks1, b1))
    ks2 = g.SplatDFJ(coulomb=g.exact(), screen=g.pairlist(-1.0, unique=True))
    E2 = ks2(g.SplatModel(basis=b2, C=C2, occupations=occ), g.refresh(ks2, b2))
    rel = abs(E1.item() - E2.item()) / abs(E2.item())
    print(f"[full-eri] CO2 M={s.M}: streamed {E1.item():.15e} screened full list "
          f"{E2.item():.15e} rel {rel:.2e}", flush=True)
    assert rel < 1e-12
    E1.backward()
    E2.backward()
    for name, a, b in (("C", C1, C2), ("centers", b1.centers, b2.centers),
                       ("quat", b1.quat, b2.quat)):
        err = rel_max(_np(a.grad), _np(b.grad))
        print(f"[full-eri] d{name} streamed vs screened rel-to-max {err:.2e}", flush=True)
        assert err < 1e-11

    class Hybrid:
        exact_exchange_fraction = 0.25

    with pytest.raises(NotImplementedError, match="M\\^4 ERI tensor"):
        g.SplatDFJ(coulomb=g.exact(), xc=Hybrid())
