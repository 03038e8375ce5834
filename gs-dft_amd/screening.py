"""Significant-pair screening on the GPU, mirroring gs_dft/screening/pairs.py.

``neighbor_pairs`` keeps the reference's contract exactly: pairs with normalised overlap
|S_ij| > eps, lexsorted by (i, j), padded at the tail with (0, 0) entries whose third output is
0, overflow keeping the pad_to largest |S| (and raising beyond twice the pad), ``eps < 0``
meaning every pair, and ``unique=True`` keeping j >= i with float weights 2 - delta_ij.
"""
from __future__ import annotations

import ctypes
import dataclasses

import torch

from . import _lib
from .basis import _has_splat_interface


def _splat_args(splats):
    q, l, c = (t.detach().contiguous() for t in (splats.quat, splats.log_scale, splats.centers))
    return q, l, c


def _pair_weights(pi: torch.Tensor, pj: torch.Tensor, unique: bool) -> torch.Tensor:
    """Third output of ``neighbor_pairs`` (gs_dft/screening/pairs.py:318-322)."""
    if not unique:
        return torch.ones(pi.shape[0], dtype=torch.bool, device=pi.device)
    return torch.where(pi == pj, 1.0, 2.0).to(torch.float64)


def pair_weight(valid: torch.Tensor, dtype=torch.float64) -> torch.Tensor:
    """``valid`` as a multiplicative factor (gs_dft/screening/pairs.py:325-327)."""
    return valid.to(dtype)


def count_significant(splats, eps: float, unique: bool = False) -> int:
    """Number of pairs with |S_ij| > eps (gs_dft/screening/pairs.py:103-118); one host sync."""
    M = splats.n_basis
    q, l, c = _splat_args(splats)
    L = _lib.lib()
    ws = _lib.workspace(_lib.size_query(L.gsdft_screen_workspace_size, M, int(unique), 0), q.device)
    n = ctypes.c_int64(0)
    _lib.check(L.gsdft_screen_count(M, _lib.ptr(q), _lib.ptr(l), _lib.ptr(c), float(eps),
                                    int(unique), _lib.ptr(ws), ws.numel(), ctypes.byref(n),
                                    _lib.stream()), "gsdft_screen_count")
    return int(n.value)


def neighbor_pairs(splats, eps: float = 1e-5, pad_to: int | None = None, row_chunk: int = 256,
                   unique: bool = False):
    """``(pi, pj, valid)`` of the significant pairs (gs_dft/screening/pairs.py:225-315).

    ``row_chunk`` only set the reference's strip residency; the GPU build tiles the candidate
    space itself, so the argument is accepted and has no effect on the result."""
    del row_chunk
    if not _has_splat_interface(splats):
        raise NotImplementedError(
            f"neighbor_pairs: {type(splats).__name__} does not expose the splat interface "
            f"(.quat / .log_scale / .centers / .n_basis)")
    M = splats.n_basis
    q, l, c = _splat_args(splats)
    dev = q.device
    n_all = M * (M + 1) // 2 if unique else M * M
    if pad_to is None:
        pad_to = n_all if eps < 0.0 else count_significant(splats, eps, unique)
        if pad_to == 0:
            z = torch.zeros(0, dtype=torch.int32, device=dev)
            return z, z, _pair_weights(z, z, unique)
    pad_to = int(pad_to)
    pi = torch.empty(pad_to, dtype=torch.int32, device=dev)
    pj = torch.empty(pad_to, dtype=torch.int32, device=dev)
    w = torch.empty(pad_to, dtype=torch.float64, device=dev)
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
