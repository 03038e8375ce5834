"""Significant-pair screening on the GPU, mirroring gs_dft/screening/pairs.py.

``neighbor_pairs`` keeps the reference's contract exactly: pairs with normalised overlap
|S_ij| > eps, lexsorted by (i, j), padded at the tail with (0, 0) entries whose third output is
0, overflow keeping the pad_to largest |S| (and raising beyond twice the pad), ``eps < 0``
meaning every pair, and ``unique=True`` keeping j >= i with float weights 2 - delta_ij.
"""
from __future__ import annotations

import ctypes
import dataclasses
import os

import torch

from . import _lib
from .basis import _has_splat_interface


def _splat_args(splats):
    q, l, c = (t.detach().contiguous() for t in (splats.quat, splats.log_scale, splats.centers))
    return q, l, c


def check_pair_indices(pi: torch.Tensor, pj: torch.Tensor, bound: int, what: str) -> None:
    """Refuses a pair list whose indices leave [0, bound): the kernels read the splat (or C) rows
    they name without a range check. One host sync."""
    if pi.shape[0] != pj.shape[0]:
        raise ValueError(f"{what}: pi and pj must have the same length")
    if pi.shape[0] == 0:
        return
    lo = int(torch.minimum(pi.min(), pj.min()))
    hi = int(torch.maximum(pi.max(), pj.max()))
    if lo < 0 or hi >= bound:
        raise ValueError(f"{what}: pair indices must lie in [0, {bound}), got [{lo}, {hi}]")


def _pair_weights(pi: torch.Tensor, pj: torch.Tensor, unique: bool) -> torch.Tensor:
    """Third output of ``neighbor_pairs`` (gs_dft/screening/pairs.py:318-322)."""
    if not unique:
        return torch.ones(pi.shape[0], dtype=torch.bool, device=pi.device)
    return torch.where(pi == pj, 1.0, 2.0).to(torch.float64)


def pair_weight(valid: torch.Tensor, dtype=torch.float64) -> torch.Tensor:
    """``valid`` as a multiplicative factor (gs_dft/screening/pairs.py:325-327)."""
    return valid.to(dtype)


SPATIAL_MAX_M = 262144
SPATIAL_AUTO_M = 4096


def use_spatial(M: int, eps: float) -> bool:
    """Whether screening takes the spatial candidate path (gs_dft/screening/pairs.py:167-222,
    284-298). Its list is bit-identical to the dense scan's, so the choice only moves time:
    ``DFTAX_PAIR_SPATIAL=1`` forces it and ``=0`` forbids it, as the reference's switch does;
    unset, it is taken from M = 4096 splats up, where it is the faster build. eps < 0 (every pair)
    and M above 262144 always scan densely."""
    if eps < 0.0 or M > SPATIAL_MAX_M:
        return False
    flag = os.environ.get("DFTAX_PAIR_SPATIAL")
    if flag is not None and flag.strip() in ("0", "1"):
        return flag.strip() == "1"
    return M >= SPATIAL_AUTO_M


def _spatial_call(splats, eps: float, unique: bool, pad_to: int, outs=(None, None, None)):
    """gsdft_screen_spatial: (status, n_sig); pad_to < 0 only counts."""
    M = splats.n_basis
    q, l, c = _splat_args(splats)
    L = _lib.lib()
    ws = _lib.workspace(_lib.size_query(L.gsdft_screen_spatial_workspace_size, M), q.device)
    n = ctypes.c_int64(0)
    rc = L.gsdft_screen_spatial(M, _lib.ptr(q), _lib.ptr(l), _lib.ptr(c), float(eps), int(unique),
                                int(pad_to), *(_lib.ptr(t) for t in outs), _lib.ptr(ws),
                                ws.numel(), ctypes.byref(n), _lib.stream())
    return rc, int(n.value)


def count_significant(splats, eps: float, unique: bool = False, spatial: bool | None = None) -> int:
    """Number of pairs with |S_ij| > eps (gs_dft/screening/pairs.py:103-118); one host sync.
    ``spatial`` None follows ``use_spatial``."""
    M = splats.n_basis
    if (use_spatial(M, eps) if spatial is None else (spatial and eps >= 0.0)):
        rc, n = _spatial_call(splats, eps, unique, -1)
        _lib.check(rc, "gsdft_screen_spatial")
        return n
    q, l, c = _splat_args(splats)
    L = _lib.lib()
    ws = _lib.workspace(_lib.size_query(L.gsdft_screen_workspace_size, M, int(unique), 0), q.device)
    n = ctypes.c_int64(0)
    _lib.check(L.gsdft_screen_count(M, _lib.ptr(q), _lib.ptr(l), _lib.ptr(c), float(eps),
                                    int(unique), _lib.ptr(ws), ws.numel(), ctypes.byref(n),
                                    _lib.stream()), "gsdft_screen_count")
    return int(n.value)


def neighbor_pairs(splats, eps: float = 1e-5, pad_to: int | None = None, row_chunk: int = 256,
                   unique: bool = False, spatial: bool | None = None):
    """``(pi, pj, valid)`` of the significant pairs (gs_dft/screening/pairs.py:225-315).

    ``row_chunk`` only set the reference's strip residency; the GPU build tiles the candidate
    space itself, so the argument is accepted and has no effect on the result. ``spatial`` (None:
    ``use_spatial``) builds from the spatial candidate superset; a list that overflows its pad
    falls back to the dense build and its keep-largest rule, as the reference's does."""
    del row_chunk
    if not _has_splat_interface(splats):
        raise NotImplementedError(
            f"neighbor_pairs: {type(splats).__name__} does not expose the splat interface "
            f"(.quat / .log_scale / .centers / .n_basis)")
    M = splats.n_basis
    q, l, c = _splat_args(splats)
    dev = q.device
    n_all = M * (M + 1) // 2 if unique else M * M
    sp = use_spatial(M, eps) if spatial is None else (bool(spatial) and eps >= 0.0)
    if pad_to is None:
        pad_to = n_all if eps < 0.0 else count_significant(splats, eps, unique, spatial=sp)
        if pad_to == 0:
            z = torch.zeros(0, dtype=torch.int32, device=dev)
            return z, z, _pair_weights(z, z, unique)
    pad_to = int(pad_to)
    pi = torch.empty(pad_to, dtype=torch.int32, device=dev)
    pj = torch.empty(pad_to, dtype=torch.int32, device=dev)
    w = torch.empty(pad_to, dtype=torch.float64, device=dev)
    if sp:
        rc, n_sp = _spatial_call(splats, eps, unique, pad_to, (pi, pj, w))
        if rc == _lib.GSDFT_OK:
            return pi, pj, (w if unique else (w != 0.0))
        if rc != _lib.GSDFT_ERR_FALLBACK:
            _lib.check(rc, "gsdft_screen_spatial")
        print(f"  [screening] spatial path overflowed (sig={n_sp}, pad={pad_to}); using the "
              f"dense scan", flush=True)
    L = _lib.lib()
    keep_cap = 0
    n_sig = ctypes.c_int64(0)
    while True:
        ws = _lib.workspace(_lib.size_query(L.gsdft_screen_workspace_size, M, int(unique),
                                            keep_cap), dev)
        rc = L.gsdft_screen_build(M, _lib.ptr(q), _lib.ptr(l), _lib.ptr(c), float(eps),
                                  int(unique), pad_to, _lib.ptr(pi), _lib.ptr(pj), _lib.ptr(w),
                                  _lib.ptr(ws), ws.numel(), ctypes.byref(n_sig), _lib.stream())
        if rc == _lib.GSDFT_ERR_WORKSPACE and keep_cap == 0 and n_sig.value > pad_to:
            keep_cap = int(n_sig.value)
            continue
        _lib.check(rc, "neighbor_pairs")
        break
    if int(n_sig.value) > pad_to:
        print(f"  [screening] pair count {int(n_sig.value)} > pad {pad_to}: keeping the {pad_to} "
              f"largest-overlap pairs (dropped {int(n_sig.value) - pad_to})", flush=True)
    valid = w if unique else (w != 0.0)
    return pi, pj, valid


def screened_overlap_pairs(splats, pi, pj) -> torch.Tensor:
    """S_ij for listed pairs (gs_dft/screening/pairs.py:373-375); values only."""
    M = splats.n_basis
    q, l, c = _splat_args(splats)
    pi, pj = _lib.i32(pi, q.device), _lib.i32(pj, q.device)
    check_pair_indices(pi, pj, M, "screened_overlap_pairs")
    S = torch.empty(pi.shape[0], dtype=torch.float64, device=q.device)
    L = _lib.lib()
    ws = _lib.workspace(_lib.size_query(L.gsdft_screen_workspace_size, M, 0, 0), q.device)
    _lib.check(L.gsdft_overlap_pairs(M, _lib.ptr(q), _lib.ptr(l), _lib.ptr(c), pi.shape[0],
                                     _lib.ptr(pi), _lib.ptr(pj), _lib.ptr(S), _lib.ptr(ws),
                                     ws.numel(), _lib.stream()), "gsdft_overlap_pairs")
    return S


@dataclasses.dataclass
class PairIndex:
    """CSR views of a pair list for the backward pass's per-splat reductions: entries grouped
    by i (row) and by j (col), each group in list order, over the first ``n_live`` entries (the
    list up to its last nonzero weight -- the padding is appended, so the rest contributes 0)."""

    n_live: int
    row_ptr: torch.Tensor
    row_perm: torch.Tensor
    col_ptr: torch.Tensor
    col_perm: torch.Tensor


def live_length(valid: torch.Tensor) -> int:
    """One past the last entry with nonzero weight (one host sync)."""
    nz = torch.nonzero(valid.reshape(-1) != 0)
    return int(nz[-1, 0].item()) + 1 if nz.numel() else 0


def build_pair_index(M: int, pi, pj, valid) -> PairIndex:
    dev = _lib.device()
    pi, pj = _lib.i32(pi, dev), _lib.i32(pj, dev)
    n = live_length(valid.to(dev))
    L = _lib.lib()
    ws = _lib.workspace(_lib.size_query(L.gsdft_pair_index_workspace_size, M, n), dev)
    row_ptr = torch.empty(M + 1, dtype=torch.int32, device=dev)
    col_ptr = torch.empty(M + 1, dtype=torch.int32, device=dev)
    row_perm = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
    col_perm = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
    _lib.check(L.gsdft_pair_index(M, n, _lib.ptr(pi), _lib.ptr(pj), _lib.ptr(row_ptr),
                                  _lib.ptr(row_perm), _lib.ptr(col_ptr), _lib.ptr(col_perm),
                                  _lib.ptr(ws), ws.numel(), _lib.stream()), "gsdft_pair_index")
    return PairIndex(n_live=n, row_ptr=row_ptr, row_perm=row_perm, col_ptr=col_ptr,
                     col_perm=col_perm)


# ------------------------------------------------------------------------ nuclear attraction

def _atoms(atom_coords, atom_charges, dev):
    R = _lib.f64(atom_coords, dev).reshape(-1, 3).contiguous()
    Z = _lib.f64(atom_charges, dev).reshape(-1).contiguous()
    if R.shape[0] != Z.shape[0] or R.shape[0] == 0:
        raise ValueError(f"atom_coords (n_atoms, 3) and atom_charges (n_atoms,) must agree and be "
                         f"non-empty, got {tuple(R.shape)} and {tuple(Z.shape)}")
    return R, Z


def density_pairs(C_orth, occ, pi, pj) -> torch.Tensor:
    """P_ij = sum_o occ_o C_io C_jo on the listed pairs (gs_dft/screening/pairs.py:383-386), without
    forming the dense M x M density; values only."""
    dev = _lib.device()
    C = _lib.f64(C_orth.detach() if isinstance(C_orth, torch.Tensor) else C_orth, dev)
    o = _lib.f64(occ.detach() if isinstance(occ, torch.Tensor) else occ, dev).reshape(-1)
    pi, pj = _lib.i32(pi, dev), _lib.i32(pj, dev)
    if C.dim() != 2 or o.shape[0] != C.shape[1]:
        raise ValueError("density_pairs: C_orth must be (M, k) with one occupation per column")
    check_pair_indices(pi, pj, C.shape[0], "density_pairs")
    out = torch.empty(pi.shape[0], dtype=torch.float64, device=dev)
    _lib.check(_lib.lib().gsdft_density_pairs(pi.shape[0], _lib.ptr(pi), _lib.ptr(pj), C.shape[1],
                                              _lib.ptr(C), _lib.ptr(o), _lib.ptr(out),
                                              _lib.stream()), "density_pairs")
    return out


def screened_nuclear_pairs(splats, pi, pj, atom_coords, atom_charges) -> torch.Tensor:
    """V_ij of the listed pairs (gs_dft/screening/pairs.py:348-370,378-380): the nuclear attraction
    -N_i N_j K sum_A Z_A v_A by the reference's 20-node Laplace rule; values only."""
    if not _has_splat_interface(splats):
        raise NotImplementedError(f"screened_nuclear_pairs: {type(splats).__name__} is not a Splat")
    M = splats.n_basis
    q, l, c = _splat_args(splats)
    dev = q.device
    pi, pj = _lib.i32(pi, dev), _lib.i32(pj, dev)
    check_pair_indices(pi, pj, M, "screened_nuclear_pairs")
    R, Z = _atoms(atom_coords, atom_charges, dev)
    n = pi.shape[0]
    V = torch.empty(n, dtype=torch.float64, device=dev)
    L = _lib.lib()
    ws = _lib.workspace(_lib.size_query(L.gsdft_external_workspace_size, M, 1, n, R.shape[0]), dev)
    _lib.check(L.gsdft_nuclear_pairs(M, _lib.ptr(q), _lib.ptr(l), _lib.ptr(c), n, _lib.ptr(pi),
                                     _lib.ptr(pj), R.shape[0], _lib.ptr(R), _lib.ptr(Z),
                                     _lib.ptr(V), _lib.ptr(ws), ws.numel(), _lib.stream()),
               "screened_nuclear_pairs")
    return V


class _ExternalFn(torch.autograd.Function):
    """E_ext = sum_a w_a P_a V_a in one library pass; with gradients requested, the same pass also
    writes dE/d(quat, log_scale, centers, C_orth, atom_coords), which the backward scales by the
    incoming cotangent."""

    @staticmethod
    def forward(ctx, quat, log_scale, centers, C, R, x):
        M, k, n, dev = x["M"], x["k"], x["n"], x["dev"]
        grads = any(ctx.needs_input_grad[:5])
        E = torch.empty((), dtype=torch.float64, device=dev)
        V = torch.empty(max(n, 1), dtype=torch.float64, device=dev)
        outs = [None] * 5
        if grads:
            outs = [torch.empty((M, 4), dtype=torch.float64, device=dev),
                    torch.empty((M, 3), dtype=torch.float64, device=dev),
                    torch.empty((M, 3), dtype=torch.float64, device=dev),
                    torch.empty((M, k), dtype=torch.float64, device=dev),
                    torch.empty_like(x["R"])]
            idx = build_pair_index(M, x["pi"][:n], x["pj"][:n], x["w"][:n])
            csr = (idx.row_ptr, idx.row_perm, idx.col_ptr, idx.col_perm)
        else:
            csr = (None, None, None, None)
        L = _lib.lib()
        ws = _lib.workspace(_lib.size_query(L.gsdft_external_workspace_size, M, k, n,
                                            x["R"].shape[0]), dev)
        q, l, c, Cd = (t.detach().contiguous() for t in (quat, log_scale, centers, C))
        _lib.check(L.gsdft_external_energy(
            M, _lib.ptr(q), _lib.ptr(l), _lib.ptr(c), k, _lib.ptr(Cd), _lib.ptr(x["occ"]), n,
            _lib.ptr(x["pi"]), _lib.ptr(x["pj"]), _lib.ptr(x["w"]), *(_lib.ptr(t) for t in csr),
            x["R"].shape[0], _lib.ptr(x["R"]), _lib.ptr(x["Z"]), _lib.ptr(E), _lib.ptr(V),
            *(_lib.ptr(t) for t in outs), _lib.ptr(ws), ws.numel(), _lib.stream()),
            "screened_external_energy")
        ctx.grads = outs if grads else None
        return E

    @staticmethod
    def backward(ctx, gE):
        if ctx.grads is None:
            return None, None, None, None, None, None
        return tuple(g * gE for g in ctx.grads) + (None,)


def screened_external_energy(splats, C_orth, occ, pi, pj, atom_coords, atom_charges, valid=None,
                             chunk: int = 8192, skip_pad: bool = False) -> torch.Tensor:
    """E_external = sum_a w_a P_a V_a over the listed pairs (gs_dft/screening/pairs.py:409-440),
    differentiable w.r.t. the splat leaves, ``C_orth`` and ``atom_coords`` (the nuclear charges are
    held constant). ``valid`` weights the entries (bool or the unique-list weights 2 - delta_ij;
    padding carries 0). ``chunk`` and ``skip_pad`` shaped the reference's XLA stream and do not
    change its value; the library always skips the appended padding."""
    del chunk, skip_pad
    if not _has_splat_interface(splats):
        raise NotImplementedError(f"screened_external_energy: {type(splats).__name__} is not a "
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
    n = live_length(w)
    check_pair_indices(pi_t[:n], pj_t[:n], M, "screened_external_energy")
    R_in = atom_coords if isinstance(atom_coords, torch.Tensor) else _lib.f64(atom_coords, dev)
    R, Z = _atoms(R_in.detach(), atom_charges, dev)
    Rg = R_in if (isinstance(R_in, torch.Tensor) and R_in.requires_grad) else R
    x = {"M": M, "k": int(C.shape[1]), "n": n, "dev": dev, "occ": occ_t, "pi": pi_t, "pj": pj_t,
         "w": w, "R": R, "Z": Z}
    return _ExternalFn.apply(splats.quat, splats.log_scale, splats.centers, C, Rg, x)
