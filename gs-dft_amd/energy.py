"""Refresh state and the DF-J energy verb, mirroring gs_dft/ks/energy.py:109-139,275-285,421-474
and the pad rule of gs_dft/ks/train.py:355-360.

``SplatDFJ`` is the part of the reference's ``SplatKS`` this path covers: it resolves
``coulomb=df()`` + ``screen=pairlist(eps)`` to ``ScreenedProductDFCoulomb`` and evaluates E_J.
``refresh`` is duck-typed on ``ks.screen`` and ``ks.coulomb`` like the reference's, so it also
accepts any SplatKS-shaped object.
"""
from __future__ import annotations

import dataclasses
import math

import torch

from . import ri as _cdf
from . import screening as _scr
from .basis import Splat, init_product_aux
from .terms import DFSpec, ExactSpec, Pairlist, ScreenedProductDFCoulomb, _make_coulomb


@dataclasses.dataclass
class SplatModel:
    """Trainable model: splats + MO coefficients (gs_dft/ks/energy.py:109-118)."""

    basis: Splat
    C: torch.Tensor
    occupations: torch.Tensor

    @property
    def n_electrons(self) -> float:
        return float(torch.sum(self.occupations))


@dataclasses.dataclass
class SplatState:
    """Refresh products for the current splats (gs_dft/ks/energy.py:121-139).

    ``pair_index`` is this library's addition: the CSR views of ``pairs`` the reverse pass uses.
    ``refresh`` fills it; when it is None it is built on first use. ``cholV_lr`` is the other
    addition: for a range-separated xc, the Cholesky factor of the erf(omega r)/r metric of
    ``aux_K`` (+ lam I), formed once per refresh like ``cholV`` instead of once per step (the
    reference forms that metric inside every long-range exchange call, ri.py:543)."""

    pairs: tuple | None = None
    aux: object | None = None
    aux_K: object | None = None
    cholV: torch.Tensor | None = None
    cells: tuple | None = None
    pair_index: _scr.PairIndex | None = None
    cholV_lr: torch.Tensor | None = None


def train_pad_to(screen: Pairlist, n0: int, n_devices: int = 1) -> int:
    """The trainer's frozen pad: ceil(pad * n0 / G) * G (gs_dft/ks/train.py:355-360)."""
    G = int(n_devices)
    return -(-int(screen.pad * n0) // G) * G


class SplatDFJ:
    """The two-electron energy of a splat model through ``coulomb=df()`` (or ``exact()``) and
    ``screen=pairlist(...)``: E_J, plus hf_coeff * E_K for a hybrid ``xc`` (an object with
    ``exact_exchange_fraction`` or ``hf_coeff``) and hf_coeff_lr * E_K[erf(omega r)/r] for a
    range-separated one (``hf_coeff_lr``, ``omega``); gs_dft/ks/energy.py:400-410 adds the same
    terms to the total."""

    def __init__(self, *, coulomb: DFSpec | ExactSpec | None = None,
                 screen: Pairlist | None = None, xc=None, mesh=None):
        if mesh is not None:
            raise NotImplementedError("mesh= shards the step across GPUs; this library runs the "
                                      "DF-J path on one GPU")
        from .terms import hf_coeff
        spec = DFSpec() if coulomb is None else coulomb
        if screen is None and not isinstance(spec, ExactSpec):
            raise NotImplementedError("the DF-J path here is the screened one: pass "
                                      "screen=pairlist(...) (eps=-1.0 keeps every pair)")
        self.screen = screen
        self.coulomb = _make_coulomb(spec, screened=screen is not None,
                                     a_x=hf_coeff(xc) if xc is not None else 0.0,
                                     a_x_lr=float(getattr(xc, "hf_coeff_lr", 0.0) or 0.0),
                                     omega=float(getattr(xc, "omega", 0.0) or 0.0),
                                     skip_pad=bool(screen is not None and screen.skip_pad))
        if screen is not None and screen.unique and self.coulomb.hf_coeff != 0.0:
            raise ValueError("pairlist(unique=True) is PBE-class only: the screened RI-K "
                             "contraction is not symmetric in the pair index")
        self.mesh = None
        self.cell_part = None

    def _check_state(self, state: SplatState) -> None:
        """gs_dft/ks/energy.py:275-285"""
        if self.screen is not None and state.pairs is None:
            raise ValueError("this SplatKS screens: pass the refresh state "
                             "(state.pairs) -- see refresh(ks, basis).")
        if isinstance(self.coulomb, ScreenedProductDFCoulomb):
            if state.aux is None:
                raise ValueError("coulomb=df() needs the frozen product aux: "
                                 "pass the refresh state -- see refresh(ks, basis).")
            if ((self.coulomb.hf_coeff != 0.0 or self.coulomb.hf_coeff_lr != 0.0)
                    and state.aux_K is None):
                raise ValueError("hybrid df() needs the K-aux: pass the refresh state "
                                 "(state.aux_K) -- see refresh(ks, basis).")

    def __call__(self, model: SplatModel, state: SplatState | None = None) -> torch.Tensor:
        state = SplatState() if state is None else state
        self._check_state(state)
        e_j, e_k = self.coulomb.energy(model.basis, model.C, None, model.occupations, state)
        e = e_j
        if self.coulomb.hf_coeff != 0.0:
            e = e + self.coulomb.hf_coeff * e_k
        if self.coulomb.hf_coeff_lr != 0.0:     # gs_dft/ks/energy.py:330,406-408
            e = e + self.coulomb.hf_coeff_lr * self.coulomb.energy_lr(
                model.basis, model.C, None, model.occupations, state)
        return e


def refresh(ks, basis: Splat, *, pad_to: int | None = None,
            like: SplatState | None = None) -> SplatState:
    """Rebuild the refresh products for the current splats (gs_dft/ks/energy.py:421-474): the
    padded pair list (``like`` inherits its pad), the frozen product aux and the Cholesky factor
    of V + lam I; plus the pair index the reverse pass reads."""
    if pad_to is None and like is not None and like.pairs is not None:
        pad_to = int(like.pairs[0].shape[0])
    if getattr(ks, "cell_part", None) is not None:
        raise NotImplementedError("the block-sparse cell grid belongs to the XC term, which this "
                                  "library does not implement")
    if getattr(ks, "mesh", None) is not None:
        raise NotImplementedError("mesh= (multi-GPU striping) is not part of this library")
    pairs = index = None
    if ks.screen is not None:
        pairs = _scr.neighbor_pairs(basis, eps=ks.screen.eps, pad_to=pad_to,
                                    unique=ks.screen.unique)
        index = _scr.build_pair_index(basis.n_basis, *pairs)
    aux = aux_K = cholV = cholV_lr = None
    coul = ks.coulomb
    if isinstance(coul, ScreenedProductDFCoulomb) or type(coul).__name__ in (
            "ScreenedProductDFCoulomb", "ProductDFCoulomb"):
        aux = init_product_aux(basis, scales=coul.scales, diagonal_only=coul.diagonal)
        if getattr(coul, "hf_coeff", 0.0) != 0.0 or getattr(coul, "hf_coeff_lr", 0.0) != 0.0:
            aux_K = aux
        cholV = _cdf.aux_cholesky(aux, coul.lam)
        if getattr(coul, "hf_coeff_lr", 0.0) != 0.0:
            cholV_lr = _cdf.aux_cholesky(aux_K, coul.lam, coul.omega)
    return SplatState(pairs=pairs, aux=aux, aux_K=aux_K, cholV=cholV, pair_index=index,
                      cholV_lr=cholV_lr)
