"""Density on a grid for the exchange-correlation term, mirroring the chunked exact density of
gs_dft/screening/grid.py:88-154: rho(r) = sum_o occ_o psi_o(r)^2 with psi = g C over the splat
values g_m(r) = N_m exp(-(r - mu_m).A_m (r - mu_m)), and grad rho and tau for the GGA and
meta-GGA variants. Values and gradients (w.r.t. the splat leaves and C; the grid is held
constant) come from ``libgsdft`` (``gsdft_grid_density`` / ``gsdft_grid_density_vjp``); the
contractions run as FP64 GEMMs.
"""
from __future__ import annotations

import torch

from . import _lib
from .basis import _has_splat_interface

_MODES = {"lda": 0, "gga": 1, "mgga": 2}


class _DensityFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, quat, log_scale, centers, C, x):
        M, k, G, dev, mode, chunk = x["M"], x["k"], x["G"], x["dev"], x["mode"], x["chunk"]
        rho = torch.empty(G, dtype=torch.float64, device=dev)
        grad = torch.empty((G, 3), dtype=torch.float64, device=dev) if mode >= 1 else None
        tau = torch.empty(G, dtype=torch.float64, device=dev) if mode == 2 else None
        L = _lib.lib()
        ws = _lib.workspace(_lib.size_query(L.gsdft_grid_density_workspace_size, M, k, chunk,
                                            mode, 0), dev)
        q, l, c, Cd = (t.detach().contiguous() for t in (quat, log_scale, centers, C))
        _lib.check(L.gsdft_grid_density(M, _lib.ptr(q), _lib.ptr(l), _lib.ptr(c), k,
                                        _lib.ptr(Cd), _lib.ptr(x["occ"]), G, _lib.ptr(x["pts"]),
                                        chunk, mode, _lib.ptr(rho), _lib.ptr(grad),
                                        _lib.ptr(tau), _lib.ptr(ws), ws.numel(), _lib.stream()),
                   "grid density")
        ctx.x = x
        ctx.save_for_backward(q, l, c, Cd)
        outs = (rho,) + ((grad,) if mode >= 1 else ()) + ((tau,) if mode == 2 else ())
        return outs

    @staticmethod
    def backward(ctx, *cots):
        x = ctx.x
        q, l, c, Cd = ctx.saved_tensors
        M, k, G, dev, mode, chunk = x["M"], x["k"], x["G"], x["dev"], x["mode"], x["chunk"]
        v = [None if t is None else t.detach().to(torch.float64).contiguous() for t in cots]
        v_rho = v[0]
        v_grad = v[1] if mode >= 1 else None
        v_tau = v[2] if mode == 2 else None
        dq = torch.empty((M, 4), dtype=torch.float64, device=dev)
        dl = torch.empty((M, 3), dtype=torch.float64, device=dev)
        dc = torch.empty((M, 3), dtype=torch.float64, device=dev)
        dC = torch.empty((M, k), dtype=torch.float64, device=dev)
        L = _lib.lib()
        ws = _lib.workspace(_lib.size_query(L.gsdft_grid_density_workspace_size, M, k, chunk,
                                            mode, 1), dev)
        _lib.check(L.gsdft_grid_density_vjp(M, _lib.ptr(q), _lib.ptr(l), _lib.ptr(c), k,
                                            _lib.ptr(Cd), _lib.ptr(x["occ"]), G,
                                            _lib.ptr(x["pts"]), chunk, mode, _lib.ptr(v_rho),
                                            _lib.ptr(v_grad), _lib.ptr(v_tau), _lib.ptr(dq),
                                            _lib.ptr(dl), _lib.ptr(dc), _lib.ptr(dC),
                                            _lib.ptr(ws), ws.numel(), _lib.stream()),
                   "grid density reverse pass")
        return dq, dl, dc, dC, None


def _density(splats, C, occ, grid_points, chunk, kind):
    if not _has_splat_interface(splats):
        raise NotImplementedError(f"grid density: {type(splats).__name__} is not a Splat")
    dev = _lib.device()
    M = splats.n_basis
    Ct = C if isinstance(C, torch.Tensor) else _lib.f64(C, dev)
    if Ct.device != dev or Ct.dtype != torch.float64:
        Ct = Ct.to(device=dev, dtype=torch.float64)
    if Ct.dim() != 2 or Ct.shape[0] != M:
        raise ValueError(f"C must be (M, k) with M = {M}, got {tuple(Ct.shape)}")
    occ_t = _lib.f64(occ.detach() if isinstance(occ, torch.Tensor) else occ, dev).reshape(-1)
    if occ_t.shape[0] != Ct.shape[1]:
        raise ValueError("occ must have one entry per column of C")
    pts = _lib.f64(grid_points.detach() if isinstance(grid_points, torch.Tensor) else grid_points,
                   dev).reshape(-1, 3).contiguous()
    chunk = int(chunk)
    if not 0 < chunk <= 65535:
        raise ValueError(f"chunk must lie in [1, 65535], got {chunk}")
    x = {"M": M, "k": int(Ct.shape[1]), "G": int(pts.shape[0]), "dev": dev, "occ": occ_t,
         "pts": pts, "mode": _MODES[kind], "chunk": chunk}
    return _DensityFn.apply(splats.quat, splats.log_scale, splats.centers, Ct, x)


def chunked_density(splats, C, occ, grid_points, chunk: int = 4096) -> torch.Tensor:
    """rho on the grid (gs_dft/screening/grid.py:140-154), differentiable w.r.t. the splat leaves
    and C; ``chunk`` only bounds the working memory."""
    return _density(splats, C, occ, grid_points, chunk, "lda")[0]


def chunked_density_and_grad(splats, C, occ, grid_points, chunk: int = 4096):
    """(rho, grad rho) on the grid (gs_dft/screening/grid.py:88-112)."""
    return _density(splats, C, occ, grid_points, chunk, "gga")


def chunked_density_grad_tau(splats, C, occ, grid_points, chunk: int = 4096):
    """(rho, grad rho, tau) on the grid (gs_dft/screening/grid.py:115-137)."""
    return _density(splats, C, occ, grid_points, chunk, "mgga")
