"""Density fitting over the screened pair list, mirroring gs_dft/coulomb/ri.py: the aux metric
and its Cholesky factor, gamma = sum_a (P|a) q_a, the robust-DF energy
E_J = 1/2 gamma^T (V + lam I)^-1 gamma, and the screened RI-K exchange energy, each with a
hand-written reverse pass.

Every value is computed by ``libgsdft``; torch autograd only routes cotangents. The aux and the
metric factor are refresh products held constant, as the reference holds its ``SplatState``
constant inside the training step (gs_dft/ks/train.py:367-373).
"""
from __future__ import annotations

import torch

from . import _lib
from .basis import IsotropicSplat, Splat
from .screening import PairIndex, build_pair_index, live_length


# ------------------------------------------------------------------------------------ metric

def _omega(omega) -> float:
    """The reference's ``omega`` argument as the library's: None / 0 select the 1/r kernel, a
    positive value the long-range kernel erf(omega r)/r."""
    w = 0.0 if not omega else float(omega)
    if not (w >= 0.0) or w == float("inf"):
        raise ValueError(f"omega must be a finite number >= 0 (or None), got {omega!r}")
    return w


def aux_metric(aux: IsotropicSplat, omega=None, *, lam: float = 0.0) -> torch.Tensor:
    """V_PQ = (P|Q) (gs_dft/coulomb/ri.py:267-275), with the kernel erf(omega r)/r when ``omega``
    is given (ri.py:70-72); ``lam`` is added to the diagonal in the same kernel (the reference's
    ``shift_diag``)."""
    w = _omega(omega)
    N = aux.n_basis
    dev = aux.log_alpha.device
    V = torch.empty((N, N), dtype=torch.float64, device=dev)
    L = _lib.lib()
    ws = _lib.workspace(_lib.size_query(L.gsdft_metric_workspace_size, N), dev)
    _lib.check(L.gsdft_aux_metric(N, _lib.ptr(aux.log_alpha), _lib.ptr(aux.centers), float(lam),
                                  w, _lib.ptr(V), _lib.ptr(ws), ws.numel(), _lib.stream()),
               "gsdft_aux_metric")
    return V


def shift_diag(V: torch.Tensor, lam: float) -> torch.Tensor:
    """``V + lam I`` by adding to the diagonal (gs_dft/coulomb/ri.py:243-250)."""
    out = V.clone()
    out.diagonal().add_(lam)
    return out


def aux_cholesky(aux: IsotropicSplat, lam: float, omega=None) -> torch.Tensor:
    """Lower Cholesky factor of V + lam I (gs_dft/coulomb/ri.py:259-264), V the metric of the
    kernel ``omega`` selects: its lower triangle formed in the factor's own buffer and factored
    in place."""
    w = _omega(omega)
    N = aux.n_basis
    dev = aux.log_alpha.device
    L = torch.empty((N, N), dtype=torch.float64, device=dev)
    Lb = _lib.lib()
    ws = _lib.workspace(_lib.size_query(Lb.gsdft_metric_workspace_size, N), dev)
    _lib.check(Lb.gsdft_aux_cholesky(N, _lib.ptr(aux.log_alpha), _lib.ptr(aux.centers),
                                     float(lam), w, _lib.ptr(L), _lib.ptr(ws), ws.numel(),
                                     _lib.stream()),
               "aux_cholesky")
    return L


# ------------------------------------------------------------------------------------ helpers

class _Inputs:
    """The device-side operands of one gamma evaluation, validated once."""

    def __init__(self, splats: Splat, C_occ, occ, aux: IsotropicSplat, pi, pj, valid, index):
        dev = _lib.device()
        self.M = splats.n_basis
        self.quat, self.log_scale, self.centers = splats.quat, splats.log_scale, splats.centers
        self.C = C_occ if isinstance(C_occ, torch.Tensor) else _lib.f64(C_occ, dev)
        if self.C.device != dev or self.C.dtype != torch.float64:
            self.C = self.C.to(device=dev, dtype=torch.float64)
        if self.C.dim() != 2 or self.C.shape[0] != self.M:
            raise ValueError(f"C_occ must be (M, k) with M = {self.M}, got {tuple(self.C.shape)}")
        self.k = int(self.C.shape[1])
        self.occ = _lib.f64(occ, dev).reshape(-1)
        if self.occ.shape[0] != self.k:
            raise ValueError("occ must have one entry per column of C_occ")
        self.aux = aux
        self.N = aux.n_basis
        self.pi, self.pj = _lib.i32(pi, dev), _lib.i32(pj, dev)
        n = self.pi.shape[0]
        if valid is None:
            valid = torch.ones(n, dtype=torch.float64, device=dev)
        self.w = _lib.f64(valid, dev).reshape(-1)
        if self.pj.shape[0] != n or self.w.shape[0] != n:
            raise ValueError("pi, pj and valid must have the same length")
        self.index = index
        self.n_live = index.n_live if index is not None else live_length(self.w)
        if index is None and self.n_live > 0:
            # a list that did not come from refresh(): every index the kernels will read must
            # name a splat (an out-of-range entry would read past the splat arrays on the GPU)
            lo = int(torch.minimum(self.pi[:self.n_live].min(), self.pj[:self.n_live].min()))
            hi = int(torch.maximum(self.pi[:self.n_live].max(), self.pj[:self.n_live].max()))
            if lo < 0 or hi >= self.M:
                raise ValueError(f"pair indices must lie in [0, {self.M}), got [{lo}, {hi}]")

    def ensure_index(self) -> PairIndex:
        if self.index is None:
            self.index = build_pair_index(self.M, self.pi, self.pj, self.w)
        return self.index


def _gamma_forward(x: _Inputs) -> torch.Tensor:
    dev = x.C.device
    gamma = torch.empty(x.N, dtype=torch.float64, device=dev)
    L = _lib.lib()
    n = x.n_live
    ws = _lib.workspace(_lib.size_query(L.gsdft_gamma_workspace_size, x.M, x.k, x.N, n), dev)
    q, l, c, C = (t.detach().contiguous() for t in (x.quat, x.log_scale, x.centers, x.C))
    _lib.check(L.gsdft_gamma(x.M, _lib.ptr(q), _lib.ptr(l), _lib.ptr(c), x.k, _lib.ptr(C),
                             _lib.ptr(x.occ), x.N, _lib.ptr(x.aux.log_alpha),
                             _lib.ptr(x.aux.centers), n, _lib.ptr(x.pi), _lib.ptr(x.pj),
                             _lib.ptr(x.w), _lib.ptr(gamma), _lib.ptr(ws), ws.numel(),
                             _lib.stream()), "df_coulomb_gamma_screened")
    return gamma


def _gamma_vjp(x: _Inputs, dgamma: torch.Tensor, dscale: torch.Tensor | None):
    """(J (pad,), dquat, dlog_scale, dcenters, dC) for the cotangent dgamma * dscale."""
    dev = x.C.device
    idx = x.ensure_index()
    n = idx.n_live
    M, k = x.M, x.k
    L = _lib.lib()
    ws = _lib.workspace(_lib.size_query(L.gsdft_gamma_vjp_workspace_size, M, k, x.N, n), dev)
    J = torch.zeros(x.pi.shape[0], dtype=torch.float64, device=dev)
    dq = torch.empty((M, 4), dtype=torch.float64, device=dev)
    dl = torch.empty((M, 3), dtype=torch.float64, device=dev)
    dc = torch.empty((M, 3), dtype=torch.float64, device=dev)
    dC = torch.empty((M, k), dtype=torch.float64, device=dev)
    dg = dgamma.detach().to(torch.float64).contiguous()
    q, l, c, C = (t.detach().contiguous() for t in (x.quat, x.log_scale, x.centers, x.C))
    _lib.check(L.gsdft_gamma_vjp(M, _lib.ptr(q), _lib.ptr(l), _lib.ptr(c), k, _lib.ptr(C),
                                 _lib.ptr(x.occ), x.N, _lib.ptr(x.aux.log_alpha),
                                 _lib.ptr(x.aux.centers), n, _lib.ptr(x.pi), _lib.ptr(x.pj),
                                 _lib.ptr(x.w), _lib.ptr(idx.row_ptr), _lib.ptr(idx.row_perm),
                                 _lib.ptr(idx.col_ptr), _lib.ptr(idx.col_perm), _lib.ptr(dg),
                                 _lib.ptr(dscale), _lib.ptr(J), _lib.ptr(dq), _lib.ptr(dl),
                                 _lib.ptr(dc), _lib.ptr(dC), _lib.ptr(ws), ws.numel(),
                                 _lib.stream()), "gamma reverse pass")
    return J, dq, dl, dc, dC


def _cho_solve(L: torch.Tensor, gamma: torch.Tensor, with_energy: bool):
    N = gamma.shape[0]
    d = torch.empty_like(gamma)
    E = torch.empty((), dtype=torch.float64, device=gamma.device) if with_energy else None
    _lib.check(_lib.lib().gsdft_cho_solve(N, _lib.ptr(L), _lib.ptr(gamma), _lib.ptr(d),
                                          _lib.ptr(E), _lib.stream()), "df_coulomb_solve")
    return d, E


# ------------------------------------------------------------------------------------ autograd

class _GammaFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, quat, log_scale, centers, C, x):
        ctx.x = x
        return _gamma_forward(x)

    @staticmethod
    def backward(ctx, dgamma):
        _J, dq, dl, dc, dC = _gamma_vjp(ctx.x, dgamma, None)
        return dq, dl, dc, dC, None


class _SolveFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gamma, L):
        d, E = _cho_solve(L.detach().contiguous(), gamma.detach().contiguous(), True)
        ctx.save_for_backward(d)
        return E

    @staticmethod
    def backward(ctx, gE):
        (d,) = ctx.saved_tensors
        return gE * d, None


class _EnergyFn(torch.autograd.Function):
    """E_J = 1/2 gamma^T (L L^T)^-1 gamma with gamma from the pair stream; the reverse pass feeds
    dE/dgamma = d = (L L^T)^-1 gamma, scaled by the incoming cotangent, straight into the
    library's gamma reverse (no torch arithmetic on the way)."""

    @staticmethod
    def forward(ctx, quat, log_scale, centers, C, x, L):
        gamma = _gamma_forward(x)
        d, E = _cho_solve(L, gamma, True)
        ctx.x = x
        ctx.save_for_backward(d)
        ctx.gamma = gamma
        return E

    @staticmethod
    def backward(ctx, gE):
        (d,) = ctx.saved_tensors
        _J, dq, dl, dc, dC = _gamma_vjp(ctx.x, d, gE.detach().to(torch.float64).contiguous())
        return dq, dl, dc, dC, None, None


# ------------------------------------------------------------------------------------ API

def df_coulomb_gamma_screened(splats: Splat, C_occ, occ, aux: IsotropicSplat, pi, pj,
                              chunk: int = 2048, valid=None, skip_pad: bool = False,
                              index: PairIndex | None = None) -> torch.Tensor:
    """gamma_P = sum_a (P|a) q_a over the listed pairs (gs_dft/coulomb/ri.py:436-469),
    differentiable w.r.t. the splat leaves and C_occ.

    ``chunk`` and ``skip_pad`` shaped the reference's XLA stream and do not change its value;
    the GPU kernels tile pairs themselves and always skip the appended padding (whose weight is
    zero, so its contribution is exactly zero either way)."""
    del chunk, skip_pad
    x = _Inputs(splats, C_occ, occ, aux, pi, pj, valid, index)
    return _GammaFn.apply(x.quat, x.log_scale, x.centers, x.C, x)


def df_coulomb_solve(gamma: torch.Tensor, aux: IsotropicSplat, lam: float = 1e-8,
                     cholV: torch.Tensor | None = None) -> torch.Tensor:
    """E_J = 1/2 gamma^T (V + lam I)^-1 gamma (gs_dft/coulomb/ri.py:472-482). Without a
    pre-factored ``cholV`` the metric is built and factored here (same value as the reference's
    dense solve to round-off)."""
    L = aux_cholesky(aux, lam) if cholV is None else cholV
    return _SolveFn.apply(gamma, L)


def df_coulomb_energy_screened(splats: Splat, C_occ, occ, aux: IsotropicSplat, pi, pj,
                               lam: float = 1e-8, chunk: int = 2048, valid=None,
                               cholV: torch.Tensor | None = None, skip_pad: bool = False,
                               index: PairIndex | None = None) -> torch.Tensor:
    """E_J^DF over the listed pairs (gs_dft/coulomb/ri.py:485-494) as one fused autograd node."""
    del chunk, skip_pad
    L = aux_cholesky(aux, lam) if cholV is None else cholV
    x = _Inputs(splats, C_occ, occ, aux, pi, pj, valid, index)
    return _EnergyFn.apply(x.quat, x.log_scale, x.centers, x.C, x, L.detach().contiguous())


def coulomb_pairs(splats: Splat, C_occ, occ, aux: IsotropicSplat, pi, pj, lam: float = 1e-8,
                  valid=None, cholV: torch.Tensor | None = None,
                  index: PairIndex | None = None) -> torch.Tensor:
    """J on the pair list, J_a = dE_J/dP_{i_a j_a} = sum_P d_P (P|a) with d = (V + lam I)^-1 gamma
    (the Coulomb matrix entries a Fock build reads; 0 on zero-weight entries)."""
    L = aux_cholesky(aux, lam) if cholV is None else cholV
    x = _Inputs(splats, C_occ, occ, aux, pi, pj, valid, index)
    gamma = _gamma_forward(x)
    d, _ = _cho_solve(L.detach().contiguous(), gamma, False)
    return _gamma_vjp(x, d, None)[0]


# ------------------------------------------------------------------------------------ RI-K

def _list_symmetric(M: int, pi: torch.Tensor, pj: torch.Tensor, w: torch.Tensor, n: int) -> bool:
    """True when the live entries of the first ``n`` come in (i, j) / (j, i) pairs of equal weight
    (the multiset of (i, j, w) equals that of (j, i, w)); then every D_P is symmetric."""
    if n == 0:
        return True
    live = w[:n] != 0
    i, j, wl = pi[:n][live].long(), pj[:n][live].long(), w[:n][live]

    def by_key_then_weight(key):
        o = torch.argsort(wl, stable=True)
        o = o[torch.argsort(key[o], stable=True)]
        return key[o], wl[o]

    k1, w1 = by_key_then_weight(i * M + j)
    k2, w2 = by_key_then_weight(j * M + i)
    return bool(torch.equal(k1, k2) and torch.equal(w1, w2))


class _ExchangeInputs:
    def __init__(self, splats: Splat, C_occ, aux: IsotropicSplat, pi, pj, valid, L, index,
                 aux_chunk: int, recompute: bool, omega: float = 0.0):
        dev = _lib.device()
        self.M = splats.n_basis
        self.quat, self.log_scale, self.centers = splats.quat, splats.log_scale, splats.centers
        C = C_occ if isinstance(C_occ, torch.Tensor) else _lib.f64(C_occ, dev)
        self.C = C.to(device=dev, dtype=torch.float64) if (C.device != dev or
                                                           C.dtype != torch.float64) else C
        if self.C.dim() != 2 or self.C.shape[0] != self.M or self.C.shape[1] == 0:
            raise ValueError(f"C_occ must be (M, k) with M = {self.M} and k >= 1, got "
                             f"{tuple(self.C.shape)}")
        self.k = int(self.C.shape[1])
        self.aux, self.N = aux, aux.n_basis
        self.L = L.detach().contiguous()
        if self.L.shape != (self.N, self.N):
            raise ValueError(f"cholV must be ({self.N}, {self.N}), got {tuple(self.L.shape)}")
        self.pi, self.pj = _lib.i32(pi, dev), _lib.i32(pj, dev)
        n = self.pi.shape[0]
        self.w = (torch.ones(n, dtype=torch.float64, device=dev) if valid is None
                  else _lib.f64(valid, dev).reshape(-1))
        if self.pj.shape[0] != n or self.w.shape[0] != n:
            raise ValueError("pi, pj and valid must have the same length")
        if n and not bool(torch.all((self.w == 0) | (self.w == 1))):
            raise ValueError("RI-K reads valid as the 0/1 mask of the ordered pair list; "
                             "unique-pair weights (pairlist(unique=True)) have no exchange "
                             "path, as in gs_dft/ks/energy.py:240-241")
        self.index = index if index is not None else build_pair_index(self.M, self.pi, self.pj,
                                                                      self.w)
        self.n = self.index.n_live
        if index is None and self.n > 0:
            lo = int(torch.minimum(self.pi[:self.n].min(), self.pj[:self.n].min()))
            hi = int(torch.maximum(self.pi[:self.n].max(), self.pj[:self.n].max()))
            if lo < 0 or hi >= self.M:
                raise ValueError(f"pair indices must lie in [0, {self.M}), got [{lo}, {hi}]")
        self.symmetric = _list_symmetric(self.M, self.pi, self.pj, self.w, self.n)
        self.aux_chunk = int(aux_chunk)
        self.recompute = int(bool(recompute))
        self.omega = float(omega)


def _exchange(x: _ExchangeInputs, grads: bool):
    """(E_K, dquat, dlog_scale, dcenters, dC) -- gradients None unless ``grads``."""
    dev = x.C.device
    M, k = x.M, x.k
    Lb = _lib.lib()
    ws = _lib.workspace(_lib.size_query(Lb.gsdft_exchange_workspace_size, M, k, x.N, x.n,
                                        int(x.symmetric), int(grads), x.aux_chunk,
                                        x.recompute), dev)
    E = torch.empty((), dtype=torch.float64, device=dev)
    out = [torch.empty(s, dtype=torch.float64, device=dev) if grads else None
           for s in ((M, 4), (M, 3), (M, 3), (M, k))]
    q, l, c, C = (t.detach().contiguous() for t in (x.quat, x.log_scale, x.centers, x.C))
    idx = x.index
    _lib.check(Lb.gsdft_exchange(M, _lib.ptr(q), _lib.ptr(l), _lib.ptr(c), k, _lib.ptr(C), x.N,
                                 _lib.ptr(x.aux.log_alpha), _lib.ptr(x.aux.centers),
                                 _lib.ptr(x.L), x.n, _lib.ptr(x.pi), _lib.ptr(x.pj),
                                 _lib.ptr(x.w), _lib.ptr(idx.row_ptr), _lib.ptr(idx.row_perm),
                                 _lib.ptr(idx.col_ptr), _lib.ptr(idx.col_perm),
                                 int(x.symmetric), x.aux_chunk, x.recompute, x.omega,
                                 _lib.ptr(E),
                                 *[_lib.ptr(t) for t in out], _lib.ptr(ws), ws.numel(),
                                 _lib.stream()), "df_exchange_energy_screened")
    return (E, *out)


class _ExchangeFn(torch.autograd.Function):
    """E_K with its gradients formed in the same library call (the reverse needs the forward's
    L^-1 D); backward scales them by the incoming cotangent."""

    @staticmethod
    def forward(ctx, quat, log_scale, centers, C, x):
        grads = any(ctx.needs_input_grad[:4])
        E, *g = _exchange(x, grads)
        if grads:
            ctx.save_for_backward(*g)
        return E

    @staticmethod
    def backward(ctx, gE):
        dq, dl, dc, dC = ctx.saved_tensors
        return gE * dq, gE * dl, gE * dc, gE * dC, None


def df_exchange_energy_screened(splats: Splat, C_occ, aux: IsotropicSplat, pi, pj,
                                lam: float = 1e-8, chunk: int = 2048, valid=None,
                                occ_chunk: int = 16, omega=None, *,
                                cholV: torch.Tensor | None = None,
                                index: PairIndex | None = None,
                                aux_chunk: int = 0, recompute: bool = False) -> torch.Tensor:
    """Screened RI-K exact-exchange energy E_K = -Tr((V + lam I)^-1 M),
    M_PQ = sum_oo' D[P,o,o'] D[Q,o,o'], D[P,o,o'] = sum over the listed pairs (i, k) of
    C_io C_ko' (P|ik) (gs_dft/coulomb/ri.py:497-544), differentiable w.r.t. the splat leaves and
    C_occ (the aux is held constant).

    ``valid`` is the 0/1 mask of the ordered pair list. ``chunk`` and ``occ_chunk`` bounded the
    reference's memory and do not change its value; ``aux_chunk`` (aux functions per pass,
    0 = automatic) and ``recompute`` (recompute the forward's (M, N, k) products in the reverse
    instead of keeping them) are this library's memory knobs, likewise without effect on the
    value. ``omega`` (> 0) evaluates the long-range exchange E_K[erf(omega r)/r] of range-separated
    hybrids (ri.py:534-544 with omega): the three-centre integrals take the 12-node rule on
    [0, omega] and the metric the erf kernel. ``cholV`` = the Cholesky factor of V + lam I for
    this ``aux`` and this ``omega`` (built here when absent)."""
    del chunk, occ_chunk
    w = _omega(omega)
    L = aux_cholesky(aux, lam, w) if cholV is None else cholV
    x = _ExchangeInputs(splats, C_occ, aux, pi, pj, valid, L, index, aux_chunk, recompute, w)
    return _ExchangeFn.apply(x.quat, x.log_scale, x.centers, x.C, x)
