"""The splat bases of the DF-J path: the full-covariance primary ``Splat`` and the isotropic
auxiliary ``IsotropicSplat``, mirroring gs_dft/basis/spectral.py:55-82 and
gs_dft/basis/isotropic.py:22-39,81-116.

Leaves are float64 tensors on the GPU; set ``requires_grad`` on them to receive gradients from
the DF-J energy. Chart quantities are computed by the library (``gsdft_splat_chart``).
"""
from __future__ import annotations

import ctypes
import dataclasses
import math

import torch

from . import _lib


@dataclasses.dataclass
class Splat:
    """Full-covariance Gaussian splats in the chart A = R(q) diag(exp l) R(q)^T
    (gs_dft/basis/spectral.py:55-82): quaternion (M,4) as (w,x,y,z), log-precision eigenvalues
    (M,3) and centres (M,3)."""

    quat: torch.Tensor
    log_scale: torch.Tensor
    centers: torch.Tensor

    def __post_init__(self):
        dev = _lib.device()
        for name in ("quat", "log_scale", "centers"):
            t = getattr(self, name)
            if not isinstance(t, torch.Tensor) or t.device != dev or t.dtype != torch.float64:
                setattr(self, name, _lib.f64(t, dev))
        M = self.centers.shape[0]
        if self.quat.shape != (M, 4) or self.log_scale.shape != (M, 3) or self.centers.shape != (M, 3):
            raise ValueError(f"Splat: expected quat (M,4), log_scale (M,3), centers (M,3); got "
                             f"{tuple(self.quat.shape)}, {tuple(self.log_scale.shape)}, "
                             f"{tuple(self.centers.shape)}")

    @property
    def n_basis(self) -> int:
        return int(self.centers.shape[0])

    def chart(self) -> tuple[torch.Tensor, torch.Tensor]:
        """(A (M,3,3), N (M)) from the library; values only (the DF-J energy carries gradients)."""
        M = self.n_basis
        A6 = torch.empty((M, 6), dtype=torch.float64, device=self.centers.device)
        N = torch.empty(M, dtype=torch.float64, device=self.centers.device)
        q, l = self.quat.detach().contiguous(), self.log_scale.detach().contiguous()
        _lib.check(_lib.lib().gsdft_splat_chart(M, _lib.ptr(q), _lib.ptr(l), _lib.ptr(A6),
                                                _lib.ptr(N), _lib.stream()), "gsdft_splat_chart")
        xx, yy, zz, xy, xz, yz = A6.unbind(1)
        A = torch.stack([torch.stack([xx, xy, xz], -1), torch.stack([xy, yy, yz], -1),
                         torch.stack([xz, yz, zz], -1)], -2)
        return A, N

    @property
    def A(self) -> torch.Tensor:
        return self.chart()[0]

    @property
    def norm(self) -> torch.Tensor:
        return self.chart()[1]


@dataclasses.dataclass
class IsotropicSplat:
    """Isotropic auxiliary Gaussians g(r) = N exp(-alpha |r - R|^2), N = (2 alpha/pi)^(3/4)
    (gs_dft/basis/isotropic.py:22-39)."""

    log_alpha: torch.Tensor
    centers: torch.Tensor

    def __post_init__(self):
        dev = _lib.device()
        self.log_alpha = _lib.f64(self.log_alpha, dev)
        self.centers = _lib.f64(self.centers, dev)
        if self.centers.shape != (self.log_alpha.shape[0], 3):
            raise ValueError("IsotropicSplat: expected log_alpha (N,) and centers (N,3)")

    @property
    def alpha(self) -> torch.Tensor:
        return torch.exp(self.log_alpha)

    @property
    def n_basis(self) -> int:
        return int(self.log_alpha.shape[0])

    @property
    def norm(self) -> torch.Tensor:
        return (2.0 * self.alpha / math.pi) ** 0.75


def _has_splat_interface(basis) -> bool:
    return all(hasattr(basis, a) for a in ("quat", "log_scale", "centers", "n_basis"))


def init_product_aux(basis: Splat, pi=None, pj=None, valid=None, *, scales=(1.0,),
                     diagonal_only: bool = True) -> IsotropicSplat:
    """Frozen density-fitting aux from the splats' pair products (gs_dft/basis/isotropic.py:81-116):
    one isotropic aux per kept pair and scale at the product centre with exponent
    det(A_i + A_j)^(1/3) * s, concatenated scale-major. With ``diagonal_only`` (or no ``pi``) the
    pairs are the self-products (i, i); otherwise they are the listed ``(pi, pj)``, and entries whose
    ``valid`` is 0 (padding) get the inert exponent s."""
    if not _has_splat_interface(basis):
        raise NotImplementedError(f"init_product_aux: {type(basis).__name__} is not a Splat")
    scales = tuple(float(s) for s in scales)
    if not scales:
        raise ValueError("init_product_aux needs at least one exponent scale")
    M = basis.n_basis
    dev = basis.centers.device
    sc = (ctypes.c_double * len(scales))(*scales)
    q, l, c = (t.detach().contiguous() for t in (basis.quat, basis.log_scale, basis.centers))
    L = _lib.lib()
    if diagonal_only or pi is None:
        la = torch.empty(len(scales) * M, dtype=torch.float64, device=dev)
        cen = torch.empty((len(scales) * M, 3), dtype=torch.float64, device=dev)
        _lib.check(L.gsdft_product_aux(M, _lib.ptr(q), _lib.ptr(l), _lib.ptr(c), sc, len(scales),
                                       _lib.ptr(la), _lib.ptr(cen), None, 0, _lib.stream()),
                   "gsdft_product_aux")
        return IsotropicSplat(log_alpha=la, centers=cen)
    from .screening import check_pair_indices
    if pj is None:
        raise ValueError("init_product_aux(diagonal_only=False) with pi needs pj as well")
    pi_t, pj_t = _lib.i32(pi, dev).reshape(-1), _lib.i32(pj, dev).reshape(-1)
    check_pair_indices(pi_t, pj_t, M, "init_product_aux")
    n = pi_t.shape[0]
    v = None
    if valid is not None:
        v = _lib.f64(torch.as_tensor(valid).to(torch.float64) if not isinstance(valid, torch.Tensor)
                     else valid.detach().to(torch.float64), dev).reshape(-1)
        if v.shape[0] != n:
            raise ValueError("init_product_aux: valid must have one entry per listed pair")
    la = torch.empty(len(scales) * n, dtype=torch.float64, device=dev)
    cen = torch.empty((len(scales) * n, 3), dtype=torch.float64, device=dev)
    ws = _lib.workspace(_lib.size_query(L.gsdft_screen_workspace_size, M, 0, 0), dev)
    _lib.check(L.gsdft_product_aux_pairs(M, _lib.ptr(q), _lib.ptr(l), _lib.ptr(c), n,
                                         _lib.ptr(pi_t), _lib.ptr(pj_t), _lib.ptr(v), sc,
                                         len(scales), _lib.ptr(la), _lib.ptr(cen), _lib.ptr(ws),
                                         ws.numel(), _lib.stream()), "gsdft_product_aux_pairs")
    return IsotropicSplat(log_alpha=la, centers=cen)
