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
