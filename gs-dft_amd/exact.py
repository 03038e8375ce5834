"""Exact Hartree energy over the significant pairs (density-fitting free), mirroring
gs_dft/coulomb/stream.py:249-320: E_J = 1/2 sum_{a,b} (a|b) Pw_a Pw_b with the pair-pair Coulomb
integral (a|b) of gs_dft/coulomb/stream.py:249-281 (the reference's 20-node rule) and
Pw_a = w_a sum_o occ_o C_{i_a o} C_{j_a o}.

Every value and gradient comes from ``libgsdft`` (``gsdft_exact_coulomb``); the cost is
O(n_pairs^2), so this is the evaluation-size path, as in the reference.
"""
from __future__ import annotations

import torch

from . import _lib
from .basis import _has_splat_interface
from .screening import PairIndex, build_pair_index, live_length, pair_weight


class _ExactFn(torch.autograd.Function):
    """One library pass: the energy (and J on the list); with gradients requested the same pass
    also writes dE/d(quat, log_scale, centers, C_orth), scaled in the backward by the incoming
    cotangent."""

    @staticmethod
    def forward(ctx, quat, log_scale, centers, C, x):
        M, k, n, dev = x["M"], x["k"], x["n"], x["dev"]
        grads = any(ctx.needs_input_grad[:4])
        E = torch.empty((), dtype=torch.float64, device=dev)
        J = torch.empty(max(n, 1), dtype=torch.float64, device=dev)
        outs = [None] * 4
        csr = (None, None, None, None)
        if grads:
            outs = [torch.empty((M, 4), dtype=torch.float64, device=dev),
                    torch.empty((M, 3), dtype=torch.float64, device=dev),
                    torch.empty((M, 3), dtype=torch.float64, device=dev),
                    torch.empty((M, k), dtype=torch.float64, device=dev)]
            idx = x["index"]
            if idx is None or idx.n_live != n:
                idx = build_pair_index(M, x["pi"][:n], x["pj"][:n], x["w"][:n])
            csr = (idx.row_ptr, idx.row_perm, idx.col_ptr, idx.col_perm)
        L = _lib.lib()
        ws = _lib.workspace(_lib.size_query(L.gsdft_exact_coulomb_workspace_size, M, k, n,
                                            int(grads)), dev)
        q, l, c, Cd = (t.detach().contiguous() for t in (quat, log_scale, centers, C))
        _lib.check(L.gsdft_exact_coulomb(
            M, _lib.ptr(q), _lib.ptr(l), _lib.ptr(c), k, _lib.ptr(Cd), _lib.ptr(x["occ"]), n,
            _lib.ptr(x["pi"]), _lib.ptr(x["pj"]), _lib.ptr(x["w"]), *(_lib.ptr(t) for t in csr),
            _lib.ptr(E), _lib.ptr(J), *(_lib.ptr(t) for t in outs), _lib.ptr(ws), ws.numel(),
            _lib.stream()), "screened_coulomb_energy")
        ctx.grads = outs if grads else None
        x["J"] = J[:n]
        return E

    @staticmethod
    def backward(ctx, gE):
        if ctx.grads is None:
            return None, None, None, None, None
        return tuple(g * gE for g in ctx.grads) + (None,)


def _inputs(splats, C_orth, occ, pi, pj, valid, index):
    if not _has_splat_interface(splats):
        raise NotImplementedError(f"screened_coulomb_energy: {type(splats).__name__} is not a "
                                  f"Splat")
    dev = _lib.device()
    M = splats.n_basis
    C = C_orth if isinstance(C_orth, torch.Tensor) else _lib.f64(C_orth, dev)
    if C.device != dev or C.dtype != torch.float64:
        C = C.to(device=dev, dtype=torch.float64)
    if C.dim() != 2 or C.shape[0] != M:
        raise ValueError(f"C_orth must be (M, k) with M = {M}, got {tuple(C.shape)}")
    occ_t = _lib.f64(occ.detach() if isinstance(occ, torch.Tensor) else occ, dev).reshape(-1)
    if occ_t.shape[0] != C.shape[1]:
        raise ValueError("occ must have one entry per column of C_orth")
    pi_t, pj_t = _lib.i32(pi, dev), _lib.i32(pj, dev)
    w = (torch.ones(pi_t.shape[0], dtype=torch.float64, device=dev) if valid is None
         else _lib.f64(pair_weight(torch.as_tensor(valid)), dev).reshape(-1))
    if pj_t.shape[0] != pi_t.shape[0] or w.shape[0] != pi_t.shape[0]:
        raise ValueError("pi, pj and valid must have the same length")
    n = index.n_live if index is not None else live_length(w)
    if n > 0 and index is None:
        lo = int(torch.minimum(pi_t[:n].min(), pj_t[:n].min()))
        hi = int(torch.maximum(pi_t[:n].max(), pj_t[:n].max()))
        if lo < 0 or hi >= M:
            raise ValueError(f"pair indices must lie in [0, {M}), got [{lo}, {hi}]")
    x = {"M": M, "k": int(C.shape[1]), "n": n, "dev": dev, "occ": occ_t, "pi": pi_t, "pj": pj_t,
         "w": w, "index": index}
    return C, x


def screened_coulomb_energy(splats, C_orth, occ, pi, pj, valid=None, bra_chunk: int = 128,
                            index: PairIndex | None = None) -> torch.Tensor:
    """Exact E_J = 1/2 sum_{a,b} (a|b) Pw_a Pw_b over the listed pairs
    (gs_dft/coulomb/stream.py:296-320), differentiable w.r.t. the splat leaves and ``C_orth``.
    ``valid`` weights the entries (bool, or 2 - delta_ij on a unique list; 0 on padding).
    ``bra_chunk`` only shaped the reference's XLA stream and does not change the value."""
    del bra_chunk
    C, x = _inputs(splats, C_orth, occ, pi, pj, valid, index)
    return _ExactFn.apply(splats.quat, splats.log_scale, splats.centers, C, x)


def screened_coulomb_J(splats, C_orth, occ, pi, pj, valid=None,
                       index: PairIndex | None = None) -> torch.Tensor:
    """Jvec_a = sum_b (a|b) Pw_b on the list (gs_dft/coulomb/stream.py:115-134; 0 on zero-weight
    entries): the exact Coulomb matrix entries a Fock build reads. Values only."""
    C, x = _inputs(splats, C_orth, occ, pi, pj, valid, index)
    with torch.no_grad():
        _ExactFn.apply(splats.quat.detach(), splats.log_scale.detach(), splats.centers.detach(),
                       C.detach(), x)
    J = torch.zeros(x["pi"].shape[0], dtype=torch.float64, device=x["dev"])
    J[:x["n"]] = x["J"]
    return J


# ------------------------------------------------------------------ density-matrix form

def make_pairs(M: int, unique: bool = True, device=None):
    """(i, j, w) over basis-function pairs (gs_dft/coulomb/stream.py:47-60): unique=True the
    M(M+1)/2 pairs i <= j in row-major order with w = 2 - delta_ij, unique=False all M^2 ordered
    pairs with w = 1. int32 indices and float64 weights on ``device``."""
    dev = _lib.device() if device is None else device
    if unique:
        ij = torch.triu_indices(M, M, device=dev)
        i, j = ij[0].to(torch.int32), ij[1].to(torch.int32)
        w = torch.where(i == j, 1.0, 2.0).to(torch.float64)
    else:
        r = torch.arange(M, dtype=torch.int32, device=dev)
        i, j = r.repeat_interleave(M), r.repeat(M)
        w = torch.ones(M * M, dtype=torch.float64, device=dev)
    return i.contiguous(), j.contiguous(), w


class _ExactDensityFn(torch.autograd.Function):
    """One library pass over the list of ``x`` with the pair densities read from P: the energy
    and, with gradients requested, dE/d(quat, log_scale, centers) and dE/dP = the Coulomb matrix
    (the reference's custom VJP, gs_dft/coulomb/stream.py:159-183), scaled in the backward by
    the incoming cotangent."""

    @staticmethod
    def forward(ctx, quat, log_scale, centers, P, x):
        M, n, dev = x["M"], x["n"], x["dev"]
        grads = any(ctx.needs_input_grad[:3])
        E = torch.empty((), dtype=torch.float64, device=dev)
        J = torch.empty(max(n, 1), dtype=torch.float64, device=dev)
        outs = [None] * 3
        csr = (None, None, None, None)
        if grads:
            outs = [torch.empty((M, 4), dtype=torch.float64, device=dev),
                    torch.empty((M, 3), dtype=torch.float64, device=dev),
                    torch.empty((M, 3), dtype=torch.float64, device=dev)]
            idx = build_pair_index(M, x["pi"], x["pj"], x["w"])
            csr = (idx.row_ptr, idx.row_perm, idx.col_ptr, idx.col_perm)
        dP = None
        if ctx.needs_input_grad[3] or x.get("want_J_matrix"):
            dP = torch.empty((M, M), dtype=torch.float64, device=dev)
        outs.append(dP)
        L = _lib.lib()
        ws = _lib.workspace(_lib.size_query(L.gsdft_exact_coulomb_workspace_size, M, 1, n,
                                            int(grads)), dev)
        q, l, c, Pd = (t.detach().contiguous() for t in (quat, log_scale, centers, P))
        _lib.check(L.gsdft_exact_coulomb_density(
            M, _lib.ptr(q), _lib.ptr(l), _lib.ptr(c), _lib.ptr(Pd), n, _lib.ptr(x["pi"]),
            _lib.ptr(x["pj"]), _lib.ptr(x["w"]), int(x["unique"]), *(_lib.ptr(t) for t in csr),
            _lib.ptr(E), _lib.ptr(J), *(_lib.ptr(t) for t in outs), _lib.ptr(ws), ws.numel(),
            _lib.stream()), "full_coulomb_energy")
        ctx.grads = outs
        x["J"] = J[:n]
        x["J_matrix"] = dP
        return E

    @staticmethod
    def backward(ctx, gE):
        return tuple(None if g is None else g * gE for g in ctx.grads) + (None,)


def _density_inputs(splats, P, unique):
    if not _has_splat_interface(splats):
        raise NotImplementedError(f"full_coulomb_energy: {type(splats).__name__} is not a Splat")
    dev = _lib.device()
    M = splats.n_basis
    Pt = P if isinstance(P, torch.Tensor) else _lib.f64(P, dev)
    if Pt.device != dev or Pt.dtype != torch.float64:
        Pt = Pt.to(device=dev, dtype=torch.float64)
    if Pt.dim() != 2 or tuple(Pt.shape) != (M, M):
        raise ValueError(f"P must be (M, M) with M = {M}, got {tuple(Pt.shape)}")
    pi, pj, w = make_pairs(M, unique, dev)
    x = {"M": M, "n": int(pi.shape[0]), "dev": dev, "pi": pi, "pj": pj, "w": w,
         "unique": bool(unique)}
    return Pt, x


def full_coulomb_energy(splats, P, bra_chunk: int = 64, unique: bool = True) -> torch.Tensor:
    """Exact E_J = 1/2 sum_pqrs (pq|rs) P_pq P_rs over every basis-function pair
    (gs_dft/coulomb/stream.py:284-287 through coulomb_energy_fused :145-187), differentiable
    w.r.t. the splat leaves and the density matrix P (M, M); the gradient w.r.t. P is the Coulomb
    matrix J (symmetric fill on the unique list), as the reference's custom VJP defines it. Only
    the upper triangle of P is read when ``unique``. O(M^4) work: the evaluation-size path.
    ``bra_chunk`` only shaped the reference's XLA stream and does not change the value."""
    del bra_chunk
    Pt, x = _density_inputs(splats, P, unique)
    return _ExactDensityFn.apply(splats.quat, splats.log_scale, splats.centers, Pt, x)


def full_coulomb_J(splats, P, bra_chunk: int = 128, unique: bool = True) -> torch.Tensor:
    """The Hartree matrix J_pq = sum_rs (pq|rs) P_rs (M, M) (gs_dft/coulomb/stream.py:189-195,
    coulomb_J_fused); values only."""
    del bra_chunk
    Pt, x = _density_inputs(splats, P, unique)
    x["want_J_matrix"] = True
    with torch.no_grad():
        _ExactDensityFn.apply(splats.quat.detach(), splats.log_scale.detach(),
                              splats.centers.detach(), Pt.detach(), x)
    return x["J_matrix"]
