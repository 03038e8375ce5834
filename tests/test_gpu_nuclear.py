"""Parity of the HIP nuclear attraction over the pair list (gs_dft/screening/pairs.py:348-440)
against the CPU oracle and the torch literal restatement, on the same seeded inputs.

Bars: V per pair within 1e-12 relative; E_ext within 1e-10 relative; gradients (splat leaves,
C and nuclear coordinates) within 1e-9 relative to the largest entry.
"""
import numpy as np
import pytest
import torch

from conftest import rel_max

pytestmark = pytest.mark.gpu

REL_E = 1e-10
REL_G = 1e-9

SMALL = [dict(M=24, k=5, n_atoms=3, seed=1), dict(M=60, k=7, n_atoms=5, seed=2, spread=4.0),
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


def _gpu_energy_grads(g, s, pi, pj, w):
    basis = g.Splat(quat=_cu(s.quat, True), log_scale=_cu(s.log_scale, True),
                    centers=_cu(s.centers, True))
    C = _cu(s.C, True)
    R = _cu(s.atoms, True)
    E = g.screened_external_energy(basis, C, s.occ, pi, pj, R, s.charges, valid=w)
    E.backward()
    return (E.item(), _np(basis.quat.grad), _np(basis.log_scale.grad), _np(basis.centers.grad),
            _np(C.grad), _np(R.grad))


@pytest.mark.parametrize("case", ["small0", "small1", "small2", "system1", "system2"])
def test_nuclear_pairs_match_oracle(g, wl, orc, cuda, case):
    s = _small(wl, SMALL[int(case[-1])]) if case.startswith("small") else wl.make_system(int(case[-1]))
    pi, pj, w, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, s.eps, None, True)
    print(f"[vne] {case}: M={s.M} n={len(pi)} atoms={len(s.charges)}", flush=True)
    basis = g.Splat(quat=_cu(s.quat), log_scale=_cu(s.log_scale), centers=_cu(s.centers))
    V = _np(g.screened_nuclear_pairs(basis, pi, pj, s.atoms, s.charges))
    ref = orc.nuclear_pairs(s.quat, s.log_scale, s.centers, pi, pj, s.atoms, s.charges)
    err = float(np.max(np.abs(V - ref) / np.abs(ref)))
    print(f"[vne] {case}: V max elementwise rel {err:.2e}")
    assert err < 1e-12


@pytest.mark.parametrize("case", [0, 1, 2])
def test_external_energy_and_gradients_match_literal(g, wl, orc, tr, cuda, case):
    """E_ext against the oracle; every gradient against autograd of the literal restatement."""
    s = _small(wl, SMALL[case])
    pi, pj, w, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, s.eps, None, True)
    got = _gpu_energy_grads(g, s, pi, pj, w)
    E_ref = orc.external_energy(s.quat, s.log_scale, s.centers, s.C, s.occ, pi, pj, w, s.atoms,
                                s.charges)
    rel = abs(got[0] - E_ref) / abs(E_ref)
    print(f"[vne] small{case}: E gpu {got[0]:.15e} oracle {E_ref:.15e} rel {rel:.2e}", flush=True)
    assert rel < REL_E
    leaves = [_t(s.quat, True), _t(s.log_scale, True), _t(s.centers, True), _t(s.C, True),
              _t(s.atoms, True)]
    Et = tr.screened_external_energy(*leaves[:4], _t(s.occ), _idx(pi), _idx(pj), _t(w),
                                     leaves[4], _t(s.charges))
    Et.backward()
    for name, a, b in zip(("quat", "log_scale", "centers", "C", "atoms"), got[1:], leaves):
        err = rel_max(a, b.grad.numpy())
        print(f"[vne] small{case}: d{name} rel-to-max {err:.2e}")
        assert err < REL_G


def test_external_energy_translation_sum_rule(g, wl, orc, cuda):
    """Moving every splat and nucleus by the same vector leaves E_ext unchanged, so the nuclear
    gradients and the splat-centre gradients sum to zero (a property of the full result)."""
    s = wl.make_system(2)
    pi, pj, w, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, s.eps, None, True)
    got = _gpu_energy_grads(g, s, pi, pj, w)
    total = got[3].sum(0) + got[5].sum(0)
    scale = np.abs(got[3]).sum() + np.abs(got[5]).sum()
    print(f"[vne] water8: |sum dE/dR + sum dE/dmu| {np.max(np.abs(total)):.2e} of {scale:.2e}")
    assert np.max(np.abs(total)) < 1e-11 * scale


def test_external_energy_unique_ordered_padding_and_determinism(g, wl, orc, cuda):
    s = _small(wl, SMALL[1])
    pu, qu, wu, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, s.eps, None, True)
    po, qo, wo, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, s.eps, None, False)
    pp, qp, wp, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, s.eps, len(pu) + 100, True)
    a = _gpu_energy_grads(g, s, pu, qu, wu)
    b = _gpu_energy_grads(g, s, po, qo, wo)
    c = _gpu_energy_grads(g, s, pp, qp, wp)
    d = _gpu_energy_grads(g, s, pu, qu, wu)
    assert abs(a[0] - b[0]) < 1e-12 * abs(a[0])
    for x, y in zip(a[1:], b[1:]):
        assert rel_max(x, y) < 1e-11
    for x, y in zip(a, c):                      # appended padding changes nothing, bit for bit
        assert np.array_equal(np.asarray(x), np.asarray(y))
    for x, y in zip(a, d):                      # repeated runs are bit-identical
        assert np.array_equal(np.asarray(x), np.asarray(y))


def test_external_energy_empty_list(g, wl, cuda):
    s = _small(wl, SMALL[0])
    z = np.zeros(0, np.int32)
    basis = g.Splat(quat=_cu(s.quat, True), log_scale=_cu(s.log_scale, True),
                    centers=_cu(s.centers, True))
    R = _cu(s.atoms, True)
    E = g.screened_external_energy(basis, _cu(s.C), s.occ, z, z, R, s.charges,
                                   valid=np.zeros(0))
    E.backward()
    assert E.item() == 0.0 and float(R.grad.abs().max()) == 0.0
    assert float(basis.centers.grad.abs().max()) == 0.0


def test_system3_energy_and_directional_derivative(g, wl, orc, cuda):
    """Alkane (M=2000, 62 nuclei): E_ext against the oracle over the full list, and the gradient's
    directional derivative (splats, C and nuclei) against central differences of the GPU energy."""
    s = wl.make_system(3)
    pi, pj, w, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, s.eps, None, True)
    basis = g.Splat(quat=_cu(s.quat, True), log_scale=_cu(s.log_scale, True),
                    centers=_cu(s.centers, True))
    C, R = _cu(s.C, True), _cu(s.atoms, True)
    E = g.screened_external_energy(basis, C, s.occ, pi, pj, R, s.charges, valid=w)
    E.backward()
    E_ref = orc.external_energy(s.quat, s.log_scale, s.centers, s.C, s.occ, pi, pj, w, s.atoms,
                                s.charges)
    print(f"[vne] system3 n={len(pi)}: E gpu {E.item():.15e} oracle {E_ref:.15e}", flush=True)
    assert abs(E.item() - E_ref) < REL_E * abs(E_ref)
    leaves = (basis.quat, basis.log_scale, basis.centers, C, R)
    gen = torch.Generator(device="cpu").manual_seed(3)
    dirs = [torch.randn(t.shape, generator=gen, dtype=torch.float64).cuda() for t in leaves]
    dd = sum((t.grad * d).sum().item() for t, d in zip(leaves, dirs))
    h = 1e-5

    def e_at(sign):
        with torch.no_grad():
            b = g.Splat(quat=basis.quat + sign * h * dirs[0],
                        log_scale=basis.log_scale + sign * h * dirs[1],
                        centers=basis.centers + sign * h * dirs[2])
            return g.screened_external_energy(b, C + sign * h * dirs[3], s.occ, pi, pj,
                                              R + sign * h * dirs[4], s.charges, valid=w).item()

    fd = (e_at(1) - e_at(-1)) / (2 * h)
    print(f"[vne] system3 directional derivative {dd:.10e} vs central difference {fd:.10e}")
    assert abs(fd - dd) < 1e-6 * max(1.0, abs(dd))


def test_out_of_range_pair_indices_are_refused(g, wl, cuda):
    """screened_overlap_pairs, density_pairs and screened_nuclear_pairs refuse an index outside
    the splat (or C) rows on the host, before any launch."""
    import pytest
    s = wl.make_small(12, 3, seed=2)
    basis = g.Splat(quat=s.quat, log_scale=s.log_scale, centers=s.centers)
    bad_i = torch.tensor([0, 12], dtype=torch.int32, device="cuda")
    bad_j = torch.tensor([-1, 3], dtype=torch.int32, device="cuda")
    ok = torch.tensor([0, 1], dtype=torch.int32, device="cuda")
    C = torch.tensor(s.C, device="cuda")
    for pi, pj in ((bad_i, ok), (ok, bad_j)):
        with pytest.raises(ValueError, match="pair indices"):
            g.screened_overlap_pairs(basis, pi, pj)
        with pytest.raises(ValueError, match="pair indices"):
            g.density_pairs(C, s.occ, pi, pj)
        with pytest.raises(ValueError, match="pair indices"):
            g.screened_nuclear_pairs(basis, pi, pj, s.atoms, s.charges)
