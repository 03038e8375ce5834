"""Parity of the HIP density on a grid (gs_dft/screening/grid.py:88-154) against the torch literal
restatement of the reference and its autograd, on the same seeded inputs.

Bars: rho, grad rho, tau within 1e-12 relative to the largest entry; gradients w.r.t. the splat
leaves and C within 1e-9 relative to the largest entry.
"""
import numpy as np
import pytest
import torch

from conftest import rel_max

pytestmark = pytest.mark.gpu

REL_V = 1e-12
REL_G = 1e-9


def _cu(a, grad=False):
    return torch.tensor(np.asarray(a), device="cuda", dtype=torch.float64).requires_grad_(grad)


def _t(x, grad=False):
    t = torch.as_tensor(np.asarray(x), dtype=torch.float64).clone()
    return t.requires_grad_(grad) if grad else t


def _np(t):
    return t.detach().cpu().numpy()


def _case(wl, M, k, n_atoms, seed, n_rad=8, n_ang=26):
    s = wl.make_small(M, k, n_atoms=n_atoms, seed=seed)
    pts = wl.atom_grid(s.atoms, n_rad=n_rad, n_ang=n_ang, r_max=8.0, seed=seed)
    return s, pts


@pytest.mark.parametrize("kind", ["lda", "gga", "mgga"])
@pytest.mark.parametrize("chunk", [4096, 37])
def test_grid_density_values_and_gradients(g, wl, tr, cuda, kind, chunk):
    s, pts = _case(wl, 30, 4, 3, seed=2)
    fn = {"lda": g.chunked_density, "gga": g.chunked_density_and_grad,
          "mgga": g.chunked_density_grad_tau}[kind]
    basis = g.Splat(quat=_cu(s.quat, True), log_scale=_cu(s.log_scale, True),
                    centers=_cu(s.centers, True))
    C = _cu(s.C, True)
    out = fn(basis, C, s.occ, pts, chunk=chunk)
    out = (out,) if kind == "lda" else out
    leaves = [_t(s.quat, True), _t(s.log_scale, True), _t(s.centers, True), _t(s.C, True)]
    ref = tr.chunked_density(*leaves, _t(s.occ), _t(pts), kind=kind)
    print(f"[grid] {kind} chunk={chunk} G={len(pts)} M={s.M} k={s.k}", flush=True)
    for name, a, b in zip(("rho", "grad", "tau"), out, ref):
        err = rel_max(_np(a), b.detach().numpy())
        print(f"[grid] {kind}: {name} rel-to-max {err:.2e}")
        assert err < REL_V
    rng = np.random.default_rng(7)
    cots = [rng.normal(size=tuple(r.shape)) for r in ref]
    E = sum((o * _cu(c)).sum() for o, c in zip(out, cots))
    E.backward()
    Et = sum((r * _t(c)).sum() for r, c in zip(ref, cots))
    Et.backward()
    for name, a, b in zip(("quat", "log_scale", "centers", "C"),
                          (basis.quat, basis.log_scale, basis.centers, C), leaves):
        err = rel_max(_np(a.grad), b.grad.numpy())
        print(f"[grid] {kind}: d{name} rel-to-max {err:.2e}")
        assert err < REL_G


def test_grid_density_system3_sampled_and_directional_derivative(g, wl, tr, cuda):
    """C20H42 (M = 2000, k = 81) on an atom-centred grid of 62 x 12 x 50 points: rho and grad rho
    on sampled points against the restatement, and the gradient's directional derivative against
    central differences of the GPU result."""
    s = wl.make_system(3)
    pts = wl.atom_grid(s.atoms, n_rad=12, n_ang=50, r_max=10.0, seed=3)
    basis = g.Splat(quat=_cu(s.quat, True), log_scale=_cu(s.log_scale, True),
                    centers=_cu(s.centers, True))
    C = _cu(s.C, True)
    rho, grad = g.chunked_density_and_grad(basis, C, s.occ, pts, chunk=1024)
    sel = np.sort(np.random.default_rng(0).choice(len(pts), 300, replace=False))
    rr, gr = tr.chunked_density(_t(s.quat), _t(s.log_scale), _t(s.centers), _t(s.C), _t(s.occ),
                                _t(pts[sel]), kind="gga")
    e1, e2 = rel_max(_np(rho)[sel], rr.numpy()), rel_max(_np(grad)[sel], gr.numpy())
    print(f"[grid] c20h42 G={len(pts)}: sampled rho {e1:.2e} grad {e2:.2e}", flush=True)
    assert e1 < REL_V and e2 < REL_V
    w = torch.tensor(np.random.default_rng(1).uniform(0.5, 1.5, len(pts)), device="cuda")
    E = (w * rho).sum() + (grad ** 2).sum() * 1e-3
    E.backward()
    leaves = (basis.quat, basis.log_scale, basis.centers, C)
    gen = torch.Generator(device="cpu").manual_seed(2)
    dirs = [torch.randn(t.shape, generator=gen, dtype=torch.float64).cuda() for t in leaves]
    dd = sum((t.grad * d).sum().item() for t, d in zip(leaves, dirs))
    h = 1e-5

    def e_at(sign):
        with torch.no_grad():
            b = g.Splat(quat=basis.quat + sign * h * dirs[0],
                        log_scale=basis.log_scale + sign * h * dirs[1],
                        centers=basis.centers + sign * h * dirs[2])
            r, gg = g.chunked_density_and_grad(b, C + sign * h * dirs[3], s.occ, pts, chunk=1024)
            return ((w * r).sum() + (gg ** 2).sum() * 1e-3).item()

    fd = (e_at(1) - e_at(-1)) / (2 * h)
    print(f"[grid] c20h42 directional derivative {dd:.10e} vs central difference {fd:.10e}")
    assert abs(fd - dd) < 1e-6 * max(1.0, abs(dd))
