"""The Coulomb / exchange plugin surface of the screened paths, mirroring gs_dft/ks/terms.py.

``df()``, ``exact()`` and ``pairlist()`` build the same frozen spec values as the reference
(terms.py:58-139) and ``_make_coulomb`` resolves ``df()`` + ``screen=pairlist(...)`` to
``ScreenedProductDFCoulomb``, ``exact()`` + ``screen=pairlist(...)`` to
``ScreenedExactCoulomb`` and ``exact()`` without a screen to ``StreamedExactCoulomb``, whose
``energy`` has the reference signature
``energy(basis, C_orth, P, occ, state) -> (E_J, E_K)`` (terms.py:146-169,180-205,236-256).
"""
from __future__ import annotations

import abc
from dataclasses import dataclass

import torch

from . import exact as _cs
from . import ri as _cdf


@dataclass(frozen=True)
class ExactSpec:
    """Exact streamed-ERI Coulomb backend (gs_dft/ks/terms.py:48-55). With a pair screen it
    resolves to ``ScreenedExactCoulomb``, without one to ``StreamedExactCoulomb`` (every basis
    pair, the density matrix P). ``chunk=None`` is the strategy default (128 screened, 64
    streamed)."""

    chunk: int | None = None


@dataclass(frozen=True)
class DFSpec:
    """Frozen pair-product density-fitting backend (gs_dft/ks/terms.py:58-65)."""

    scales: tuple = (1.0,)
    diagonal: bool = True
    lam: float = 1e-8
    chunk: int = 2048


SCREEN_PAD = 2.0
"""Default pair-list pad multiplier (gs_dft/ks/terms.py:68)."""


@dataclass(frozen=True)
class Pairlist:
    """Significant-overlap pair screening spec (gs_dft/ks/terms.py:73-89)."""

    eps: float = 1e-7
    pad: float = SCREEN_PAD
    unique: bool = False
    skip_pad: bool = False


def exact(*, chunk: int | None = None) -> ExactSpec:
    return ExactSpec(chunk=chunk)


def df(*, scales: tuple = (1.0,), diagonal: bool = True, lam: float = 1e-8,
       chunk: int = 2048) -> DFSpec:
    """Density-fitted Coulomb on the frozen self-product aux (gs_dft/ks/terms.py:108-124)."""
    if not scales:
        raise ValueError("df(scales=...) needs at least one exponent scale.")
    return DFSpec(scales=tuple(float(s) for s in scales), diagonal=bool(diagonal),
                  lam=float(lam), chunk=int(chunk))


def pairlist(eps: float = 1e-7, *, pad: float = SCREEN_PAD, unique: bool = False,
             skip_pad: bool = False) -> Pairlist:
    """Screen to the pairs with |S_ij| > eps (gs_dft/ks/terms.py:127-139)."""
    return Pairlist(eps=float(eps), pad=float(pad), unique=bool(unique), skip_pad=bool(skip_pad))


class CoulombTerm(abc.ABC):
    """``(E_J, E_K)`` of a splat density (gs_dft/ks/terms.py:146-177)."""

    hf_coeff: float = 0.0
    hf_coeff_lr: float = 0.0
    omega: float = 0.0

    @abc.abstractmethod
    def energy(self, basis, C_orth, P, occ, state) -> tuple[torch.Tensor, torch.Tensor]:
        raise NotImplementedError

    def energy_lr(self, basis, C_orth, P, occ, state) -> torch.Tensor:
        return torch.zeros((), dtype=torch.float64, device=C_orth.device)


@dataclass(frozen=True)
class ScreenedProductDFCoulomb(CoulombTerm):
    """Frozen pair-product RI-J / RI-K over the significant pairs (gs_dft/ks/terms.py:236-264).
    E_K (unscaled) is evaluated when ``hf_coeff`` != 0, on the K-aux ``state.aux_K``; the
    long-range exchange E_K[erf(omega r)/r] of range-separated hybrids when ``hf_coeff_lr`` != 0
    (``energy_lr``)."""

    hf_coeff: float = 0.0
    hf_coeff_lr: float = 0.0
    omega: float = 0.0
    lam: float = 1e-8
    chunk: int = 2048
    scales: tuple = (1.0,)
    diagonal: bool = True
    skip_pad: bool = False

    def energy(self, basis, C_orth, P, occ, state):
        pi, pj, valid = state.pairs
        e_j = _cdf.df_coulomb_energy_screened(basis, C_orth, occ, state.aux, pi, pj,
                                              lam=self.lam, chunk=self.chunk, valid=valid,
                                              cholV=state.cholV, skip_pad=self.skip_pad,
                                              index=getattr(state, "pair_index", None))
        if self.hf_coeff != 0.0:
            same = state.aux_K is state.aux
            e_k = _cdf.df_exchange_energy_screened(
                basis, C_orth, state.aux_K, pi, pj, lam=self.lam, chunk=self.chunk, valid=valid,
                cholV=state.cholV if same else None,
                index=getattr(state, "pair_index", None))
        else:
            e_k = torch.zeros((), dtype=torch.float64, device=e_j.device)
        return e_j, e_k

    def energy_lr(self, basis, C_orth, P, occ, state):
        """Unscaled E_K[erf(omega r)/r] on ``state.aux_K`` (gs_dft/ks/terms.py:258-264), with the
        erf metric's factor from ``state.cholV_lr`` (refresh forms it) or, without one, formed
        here as the reference forms its metric inside the call."""
        if self.hf_coeff_lr == 0.0:
            return torch.zeros((), dtype=torch.float64, device=C_orth.device)
        pi, pj, valid = state.pairs
        return _cdf.df_exchange_energy_screened(
            basis, C_orth, state.aux_K, pi, pj, lam=self.lam, chunk=self.chunk, valid=valid,
            omega=self.omega, cholV=getattr(state, "cholV_lr", None),
            index=getattr(state, "pair_index", None))


@dataclass(frozen=True)
class ScreenedExactCoulomb(CoulombTerm):
    """Exact streamed ERI over the significant pairs, density-fitting free
    (gs_dft/ks/terms.py:193-205); pure functionals only (no screened exact exchange)."""

    hf_coeff: float = 0.0
    chunk: int = 128

    def energy(self, basis, C_orth, P, occ, state):
        pi, pj, valid = state.pairs
        e_j = _cs.screened_coulomb_energy(basis, C_orth, occ, pi, pj, valid=valid,
                                          bra_chunk=self.chunk,
                                          index=getattr(state, "pair_index", None))
        return e_j, torch.zeros((), dtype=torch.float64, device=e_j.device)


@dataclass(frozen=True)
class StreamedExactCoulomb(CoulombTerm):
    """Exact E_J over every basis pair from the density matrix P (gs_dft/ks/terms.py:180-191:
    full_coulomb_energy, the path ``evaluate()`` reports, gs_dft/ks/train.py:554); pure
    functionals only here (the reference's hybrid branch builds the dense M^4 ERI tensor for
    E_K, which this library does not form). With P None it is formed from C_orth and occ as the
    reference's SplatKS does (gs_dft/ks/energy.py:335)."""

    hf_coeff: float = 0.0
    chunk: int = 64

    def energy(self, basis, C_orth, P, occ, state):
        if P is None:
            occ_t = torch.as_tensor(occ, dtype=torch.float64, device=C_orth.device)
            P = (C_orth * occ_t) @ C_orth.T
        e_j = _cs.full_coulomb_energy(basis, P, bra_chunk=self.chunk)
        return e_j, torch.zeros((), dtype=torch.float64, device=e_j.device)


def hf_coeff(xc) -> float:
    """Exact-exchange fraction a_x of a functional (gs_dft/ks/terms.py:267-270)."""
    a = getattr(xc, "exact_exchange_fraction", None)
    return float(a) if a is not None else float(getattr(xc, "hf_coeff", 0.0))


def _make_coulomb(spec, screened: bool, a_x: float = 0.0, a_x_lr: float = 0.0,
                  omega: float = 0.0, skip_pad: bool = False) -> CoulombTerm:
    """Resolve a spec into its term (gs_dft/ks/terms.py:273-301). The screened strategies
    (DF-J and exact) and the streamed exact one are implemented here; the others raise with the
    reason."""
    if isinstance(spec, DFSpec):
        if not screened:
            raise NotImplementedError("dense (unscreened) DF is not part of this library; pass "
                                      "screen=pairlist(eps=-1.0) for the full pair list")
        return ScreenedProductDFCoulomb(hf_coeff=a_x, hf_coeff_lr=a_x_lr, omega=omega,
                                        lam=spec.lam, chunk=spec.chunk, scales=spec.scales,
                                        diagonal=spec.diagonal, skip_pad=bool(skip_pad))
    if isinstance(spec, ExactSpec):
        if a_x_lr != 0.0:
            raise ValueError("coulomb=exact() has no range-separated exchange path; a functional "
                             f"with hf_coeff_lr={a_x_lr} needs coulomb=df()")
        if not screened:
            if a_x != 0.0:
                raise NotImplementedError(
                    "StreamedExactCoulomb's exact exchange needs the dense M^4 ERI tensor "
                    "(gs_dft/ks/terms.py:187-189), which this library does not form; use "
                    "coulomb=df() (screened RI-K) for hybrids")
            return StreamedExactCoulomb(hf_coeff=0.0, chunk=64 if spec.chunk is None else spec.chunk)
        if a_x != 0.0:
            raise ValueError("screened exact Coulomb has no exact-exchange path; use a pure "
                             "functional or coulomb=df() (screened RI-K) for hybrids.")
        return ScreenedExactCoulomb(hf_coeff=0.0, chunk=128 if spec.chunk is None else spec.chunk)
    raise TypeError(f"coulomb must come from exact() or df(), got {spec!r}")
