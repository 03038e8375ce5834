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
