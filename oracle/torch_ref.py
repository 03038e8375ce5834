"""Literal float64 restatement of the reference DF-J kernels in PyTorch (CPU), differentiable by
autograd.

TEST INFRASTRUCTURE ONLY. Where the C oracle rewrites the (iso aux | full pair) node sum in
rotation invariants, this module follows the reference line by line: an ``eigh`` of the pair
precision, the rotated displacement squared, and the per-axis node loop. Autograd through it
plays the role of JAX reverse mode, so it pins both the C oracle's forward and its hand-written
reverse pass. Use it on small systems only (it materialises the (N_aux, n_pair) block).
"""
from __future__ import annotations

import math

import numpy as np
import torch

PI = math.pi


def quad_table(n: int = 20):
    """gs_dft/integrals/dense.py:46-53 -- numpy leggauss mapped to [0, inf) by t = s/(1-s)."""
    nodes_01, weights_01 = np.polynomial.legendre.leggauss(n)
    s = (nodes_01 + 1.0) / 2.0
    w_s = weights_01 / 2.0
    t = s / (1.0 - s)
    jacobian = 1.0 / (1.0 - s) ** 2
    return np.asarray(t, dtype=np.float64), np.asarray(w_s * jacobian, dtype=np.float64)


_QT, _QW = quad_table(20)
QUAD_T_LIST = [float(t) for t in _QT]
QUAD_W_LIST = [float(w) for w in _QW]


def quat_to_rotation(q):
    """gs_dft/basis/spectral.py:33-40"""
    q = q / (torch.linalg.norm(q, dim=-1, keepdim=True) + 1e-12)
    w, x, y, z = q[..., 0], q[..., 1], q[..., 2], q[..., 3]
    r0 = torch.stack([1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)], dim=-1)
    r1 = torch.stack([2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)], dim=-1)
    r2 = torch.stack([2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)], dim=-1)
    return torch.stack([r0, r1, r2], dim=-2)


def splat_A(quat, log_scale):
    """gs_dft/basis/spectral.py:72-76"""
    R = quat_to_rotation(quat)
    a = torch.exp(log_scale)
    return torch.einsum("mij,mj,mkj->mik", R, a, R)


def splat_norm(log_scale):
    """gs_dft/basis/spectral.py:79-82"""
    detA = torch.exp(torch.sum(log_scale, dim=-1))
    return (8.0 * detA / PI ** 3) ** 0.25


def det3(A):
    """gs_dft/integrals/linalg3.py:17-22"""
    return (A[..., 0, 0] * (A[..., 1, 1] * A[..., 2, 2] - A[..., 1, 2] * A[..., 2, 1])
            - A[..., 0, 1] * (A[..., 1, 0] * A[..., 2, 2] - A[..., 1, 2] * A[..., 2, 0])
            + A[..., 0, 2] * (A[..., 1, 0] * A[..., 2, 1] - A[..., 1, 1] * A[..., 2, 0]))


def adj3(A):
    """gs_dft/integrals/linalg3.py:26-41"""
    c00 = A[..., 1, 1] * A[..., 2, 2] - A[..., 1, 2] * A[..., 2, 1]
    c01 = A[..., 0, 2] * A[..., 2, 1] - A[..., 0, 1] * A[..., 2, 2]
    c02 = A[..., 0, 1] * A[..., 1, 2] - A[..., 0, 2] * A[..., 1, 1]
    c10 = A[..., 1, 2] * A[..., 2, 0] - A[..., 1, 0] * A[..., 2, 2]
    c11 = A[..., 0, 0] * A[..., 2, 2] - A[..., 0, 2] * A[..., 2, 0]
    c12 = A[..., 0, 2] * A[..., 1, 0] - A[..., 0, 0] * A[..., 1, 2]
    c20 = A[..., 1, 0] * A[..., 2, 1] - A[..., 1, 1] * A[..., 2, 0]
    c21 = A[..., 0, 1] * A[..., 2, 0] - A[..., 0, 0] * A[..., 2, 1]
    c22 = A[..., 0, 0] * A[..., 1, 1] - A[..., 0, 1] * A[..., 1, 0]
    return torch.stack([torch.stack([c00, c01, c02], dim=-1),
                        torch.stack([c10, c11, c12], dim=-1),
                        torch.stack([c20, c21, c22], dim=-1)], dim=-2)


def solve3(A, b):
    """gs_dft/integrals/linalg3.py:49-51"""
    return torch.einsum("...kl,...l->...k", adj3(A), b) / det3(A)[..., None]


def full_pair_quantities(A, mu, N, pi, pj):
    """gs_dft/coulomb/stream.py:203-215"""
    Ai, Aj = A[pi], A[pj]
    mui, muj = mu[pi], mu[pj]
    Aij = Ai + Aj
    rhs = torch.einsum("pkl,pl->pk", Ai, mui) + torch.einsum("pkl,pl->pk", Aj, muj)
    Pa = solve3(Aij, rhs)
    d = mui - muj
    Ajd = torch.einsum("pkl,pl->pk", Aj, d)
    AiAinvAjd = torch.einsum("pkl,pl->pk", Ai, solve3(Aij, Ajd))
    K = torch.exp(-torch.sum(d * AiAinvAjd, dim=-1))
    return Aij, Pa, N[pi] * N[pj] * K


def full_overlap_pairs(quat, log_scale, centers, pi, pj):
    """gs_dft/screening/pairs.py:342-345"""
    A, N = splat_A(quat, log_scale), splat_norm(log_scale)
    Aij, _, NK = full_pair_quantities(A, centers, N, pi, pj)
    return NK * PI ** 1.5 / torch.sqrt(det3(Aij))


def init_product_aux(quat, log_scale, centers, scales=(1.0,)):
    """gs_dft/basis/isotropic.py:81-116 (diagonal_only=True) -> (log_alpha, centers)."""
    A, N = splat_A(quat, log_scale), splat_norm(log_scale)
    idx = torch.arange(A.shape[0])
    Aij, Pa, _ = full_pair_quantities(A, centers, N, idx, idx)
    alpha0 = det3(Aij) ** (1.0 / 3.0)
    log_alpha = torch.cat([torch.log(alpha0 * float(s)) for s in scales])
    return log_alpha, torch.cat([Pa for _ in scales], dim=0)


def boys0(T):
    """F0(T) = 0.5 sqrt(pi/T) erf(sqrt(T)) with the series 1 - T/3 below 1e-12."""
    Ts = torch.where(T < 1e-12, torch.ones_like(T), T)
    big = 0.5 * torch.sqrt(PI / Ts) * torch.special.erf(torch.sqrt(Ts))
    return torch.where(T < 1e-12, 1.0 - T / 3.0, big)


def coulomb_block(g1, P1, KN1, g2, P2, KN2, omega=None):
    """gs_dft/coulomb/ri.py:63-76"""
    gab = g1[:, None] * g2[None, :]
    gsum = g1[:, None] + g2[None, :]
    PQ2 = torch.sum((P1[:, None, :] - P2[None, :, :]) ** 2, dim=-1)
    rho = gab / gsum
    T = rho * PQ2
    if omega:
        z = (omega ** 2) / (omega ** 2 + rho)
        F0 = torch.sqrt(z) * boys0(z * T)
    else:
        F0 = boys0(T)
    coulomb = 2.0 * PI ** 2.5 / (gab * torch.sqrt(gsum)) * F0
    return (KN1[:, None] * KN2[None, :]) * coulomb


def aux_quantities(log_alpha, centers):
    """gs_dft/basis/isotropic.py:30-39 and gs_dft/coulomb/ri.py:238-240"""
    beta = torch.exp(log_alpha)
    return beta, centers, (2.0 * beta / PI) ** 0.75


def aux_metric(log_alpha, centers, omega=None):
    """gs_dft/coulomb/ri.py:267-275"""
    b, R, n = aux_quantities(log_alpha, centers)
    return coulomb_block(b, R, n, b, R, n, omega)


def isobra_nodes(beta, dp2, Lam, table=None):
    """gs_dft/coulomb/ri.py:167-185, the static node unroll (``table`` = (t list, w list) to
    integrate with another rule; the reference's 20 nodes by default)."""
    t_list, w_list = (QUAD_T_LIST, QUAD_W_LIST) if table is None else table
    b = beta[:, None]
    L0, L1, L2 = Lam[None, :, 0], Lam[None, :, 1], Lam[None, :, 2]
    coul = torch.zeros((beta.shape[0], Lam.shape[0]), dtype=beta.dtype)
    for t, w in zip(t_list, w_list):
        t2 = t * t
        G0 = b * L0 + t2 * (b + L0)
        G1 = b * L1 + t2 * (b + L1)
        G2 = b * L2 + t2 * (b + L2)
        invp = 1.0 / (G0 * G1 * G2)
        num = b * (L0 * dp2[..., 0] * G1 * G2
                   + L1 * dp2[..., 1] * G0 * G2
                   + L2 * dp2[..., 2] * G0 * G1)
        coul = coul + w * torch.sqrt(invp) * torch.exp(-t2 * num * invp)
    return coul


def full_isobra_block(beta, R_aux, KN_aux, A_pair, P_pair, KN_pair, table=None):
    """gs_dft/coulomb/ri.py:126-151"""
    Lam, U = torch.linalg.eigh(A_pair)
    d = R_aux[:, None, :] - P_pair[None, :, :]
    dp2 = torch.einsum("bki,abk->abi", U, d) ** 2
    coul = isobra_nodes(beta, dp2, Lam, table)
    pref = 2.0 * PI ** 3 / math.sqrt(PI)
    return (KN_aux[:, None] * KN_pair[None, :]) * pref * coul


def gamma_screened(quat, log_scale, centers, C, occ, log_alpha, aux_centers, pi, pj, valid,
                   chunk=2048):
    """gs_dft/coulomb/ri.py:436-469 (chunked, no remat needed for the values)."""
    A, N = splat_A(quat, log_scale), splat_norm(log_scale)
    aux_q = aux_quantities(log_alpha, aux_centers)
    n = pi.shape[0]
    gamma = torch.zeros(log_alpha.shape[0], dtype=torch.float64)
    for s in range(0, n, chunk):
        ci, cj, cv = pi[s:s + chunk], pj[s:s + chunk], valid[s:s + chunk]
        q = cv.to(torch.float64) * torch.sum(occ[None, :] * C[ci] * C[cj], dim=1)
        block = full_isobra_block(*aux_q, *full_pair_quantities(A, centers, N, ci, cj))
        gamma = gamma + block @ q
    return gamma


def screened_exchange_energy(quat, log_scale, centers, C, log_alpha, aux_centers, pi, pj, valid,
                             lam, chunk=2048, occ_chunk=16, table=None, omega=None):
    """gs_dft/coulomb/ri.py:497-544 as written: per occupied chunk, the pair stream builds
    D[:, chunk, :] (ri.py:524-531) and M += D D^T (ri.py:532); E_K = -tr(solve(V + lam I, M)).
    ``table`` replaces the 20-node rule of the three-centre block (for limit checks); ``omega``
    selects the erf metric (ri.py:543) -- the long-range exchange passes the segment rule on
    [0, omega] as ``table`` together with it."""
    A, N = splat_A(quat, log_scale), splat_norm(log_scale)
    aux_q = aux_quantities(log_alpha, aux_centers)
    Na, n_occ, n = log_alpha.shape[0], C.shape[1], pi.shape[0]
    mask = valid != 0
    Mmat = torch.zeros((Na, Na), dtype=torch.float64)
    for o0 in range(0, n_occ, occ_chunk):
        o1 = min(n_occ, o0 + occ_chunk)
        D = torch.zeros((Na, o1 - o0, n_occ), dtype=torch.float64)
        for s in range(0, n, chunk):
            ci, cj, cv = pi[s:s + chunk], pj[s:s + chunk], mask[s:s + chunk]
            block = full_isobra_block(*aux_q, *full_pair_quantities(A, centers, N, ci, cj), table)
            Ci = torch.where(cv[:, None], C[ci][:, o0:o1], torch.zeros((), dtype=torch.float64))
            D = D + torch.einsum("Ap,po,pq->Aoq", block, Ci, C[cj])
        Mmat = Mmat + torch.einsum("Aoq,Boq->AB", D, D)
    V = aux_metric(log_alpha, aux_centers, omega)
    Vs = V + lam * torch.eye(Na, dtype=torch.float64)
    return -torch.trace(torch.linalg.solve(Vs, Mmat))


def coulomb_solve(gamma, L):
    """gs_dft/coulomb/ri.py:479 -- 0.5 gamma^T cho_solve((L, lower), gamma)."""
    d = torch.cholesky_solve(gamma[:, None], L, upper=False)[:, 0]
    return 0.5 * torch.dot(gamma, d)


def as_t(x, requires_grad=False, dtype=torch.float64):
    t = torch.as_tensor(np.asarray(x), dtype=dtype).clone()
    return t.requires_grad_(requires_grad) if requires_grad else t


def full_nuclear_pairs(quat, log_scale, centers, pi, pj, atom_coords, atom_charges, table=None):
    """gs_dft/screening/pairs.py:348-370, node by node: B = A_ij + t^2 I, one reciprocal of det B
    per pair, the adjugate form of the exponent (``table`` = (t list, w list) for another rule)."""
    t_list, w_list = (QUAD_T_LIST, QUAD_W_LIST) if table is None else table
    A, N = splat_A(quat, log_scale), splat_norm(log_scale)
    Aij, mup, NK = full_pair_quantities(A, centers, N, pi, pj)
    d = mup[:, None, :] - atom_coords[None, :, :]
    d2 = torch.sum(d * d, dim=-1)
    eye = torch.eye(3, dtype=torch.float64)
    vA = torch.zeros(d2.shape, dtype=torch.float64)
    for t, w in zip(t_list, w_list):
        t2 = t * t
        B = Aij + t2 * eye
        invdet = 1.0 / det3(B)
        qf = torch.einsum("pak,pkl,pal->pa", d, adj3(B), d)
        expo = t2 * d2 - (t2 * t2) * qf * invdet[:, None]
        vA = vA + (w * PI ** 1.5) * torch.sqrt(invdet)[:, None] * torch.exp(-expo)
    vA = (2.0 / math.sqrt(PI)) * vA
    return -torch.sum(atom_charges[None, :] * vA, dim=1) * NK


def screened_external_energy(quat, log_scale, centers, C, occ, pi, pj, valid, atom_coords,
                             atom_charges):
    """gs_dft/screening/pairs.py:409-440 (one chunk: the sum does not depend on chunking)."""
    Pp = valid.to(torch.float64) * torch.sum(occ[None, :] * C[pi] * C[pj], dim=1)
    V = full_nuclear_pairs(quat, log_scale, centers, pi, pj, atom_coords, atom_charges)
    return torch.sum(Pp * V)


def inv3(A):
    """gs_dft/integrals/linalg3.py:44-46"""
    return adj3(A) / det3(A)[..., None, None]


def full_eri_block_schur(quat, log_scale, centers, bra_i, bra_j, ket_i, ket_j, table=None):
    """gs_dft/coulomb/stream.py:249-281, node by node (``table`` = (t list, w list) for another
    rule)."""
    t_list, w_list = (QUAD_T_LIST, QUAD_W_LIST) if table is None else table
    A, N = splat_A(quat, log_scale), splat_norm(log_scale)
    Aa, Pa, KNa = full_pair_quantities(A, centers, N, bra_i, bra_j)
    Ab, Pb, KNb = full_pair_quantities(A, centers, N, ket_i, ket_j)
    va = torch.einsum("akl,al->ak", Aa, Pa)
    vb = torch.einsum("bkl,bl->bk", Ab, Pb)
    cv = torch.sum(Pa * va, -1)[:, None] + torch.sum(Pb * vb, -1)[None, :]
    eye = torch.eye(3, dtype=torch.float64)
    coul = torch.zeros((Aa.shape[0], Ab.shape[0]), dtype=torch.float64)
    for t, w_q in zip(t_list, w_list):
        t2 = t * t
        X = Aa + t2 * eye
        Xinv = inv3(X)
        u = torch.einsum("akl,al->ak", Xinv, va)
        vau = torch.sum(va * u, -1)
        Y = Ab + t2 * eye
        S = Y[None, :] - t2 * t2 * Xinv[:, None]
        w = t2 * u[:, None, :] + vb[None, :, :]
        z = solve3(S, w)
        quad = cv - (vau[:, None] + torch.sum(w * z, -1))
        detG = det3(X)[:, None] * det3(S)
        I_t = PI ** 3 / torch.sqrt(detG) * torch.exp(-quad)
        coul = coul + w_q * (2.0 / math.sqrt(PI)) * I_t
    return (KNa[:, None] * KNb[None, :]) * coul


def screened_coulomb_energy(quat, log_scale, centers, C, occ, pi, pj, valid):
    """gs_dft/coulomb/stream.py:296-320 (one bra chunk: the sum does not depend on chunking)."""
    Pw = valid.to(torch.float64) * torch.sum(occ[None, :] * C[pi] * C[pj], dim=1)
    block = full_eri_block_schur(quat, log_scale, centers, pi, pj, pi, pj)
    return 0.5 * torch.sum((block @ Pw) * Pw)


def make_pairs(M, unique=True):
    """gs_dft/coulomb/stream.py:47-60"""
    if not unique:
        i = torch.arange(M).repeat_interleave(M)
        j = torch.arange(M).repeat(M)
        return i, j, torch.ones(M * M, dtype=torch.float64)
    i, j = torch.triu_indices(M, M)
    return i, j, torch.where(i == j, 1.0, 2.0).to(torch.float64)


def full_coulomb_energy(quat, log_scale, centers, P, unique=True):
    """gs_dft/coulomb/stream.py:145-151,284-287 (coulomb_energy_fused's value; one bra chunk)."""
    pi, pj, w = make_pairs(P.shape[0], unique)
    Pw = P[pi, pj] * w
    block = full_eri_block_schur(quat, log_scale, centers, pi, pj, pi, pj)
    return 0.5 * torch.sum((block @ Pw) * Pw)


def full_eval_block(A, centers, norm, pts):
    """gs_dft/screening/grid.py:52-70: splat values g (n, M) and gradients dg (n, M, 3) at pts."""
    dx = pts[:, None, 0] - centers[None, :, 0]
    dy = pts[:, None, 1] - centers[None, :, 1]
    dz = pts[:, None, 2] - centers[None, :, 2]
    a00, a11, a22 = A[None, :, 0, 0], A[None, :, 1, 1], A[None, :, 2, 2]
    a01, a02, a12 = A[None, :, 0, 1], A[None, :, 0, 2], A[None, :, 1, 2]
    Adr0 = a00 * dx + a01 * dy + a02 * dz
    Adr1 = a01 * dx + a11 * dy + a12 * dz
    Adr2 = a02 * dx + a12 * dy + a22 * dz
    g = norm[None, :] * torch.exp(-(dx * Adr0 + dy * Adr1 + dz * Adr2))
    dg = -2.0 * torch.stack([Adr0, Adr1, Adr2], dim=-1) * g[:, :, None]
    return g, dg


def chunked_density(quat, log_scale, centers, C, occ, pts, kind="gga", chunk=4096):
    """gs_dft/screening/grid.py:88-154: (rho,), (rho, grad) or (rho, grad, tau) for kind
    lda / gga / mgga, chunked over the points (the values do not depend on the chunking)."""
    A, N = splat_A(quat, log_scale), splat_norm(log_scale)
    out = {"rho": [], "grad": [], "tau": []}
    for s0 in range(0, pts.shape[0], chunk):
        p = pts[s0:s0 + chunk]
        g, dg = full_eval_block(A, centers, N, p)
        psi = g @ C
        out["rho"].append(torch.sum(occ[None, :] * psi ** 2, dim=1))
        if kind == "gga":
            phi = (psi * occ[None, :]) @ C.T
            out["grad"].append(2.0 * torch.einsum("gm,gmd->gd", phi, dg))
        elif kind == "mgga":
            dpsi = torch.einsum("gmd,mn->gnd", dg, C)
            out["grad"].append(2.0 * torch.einsum("n,gn,gnd->gd", occ, psi, dpsi))
            out["tau"].append(0.5 * torch.einsum("n,gnd,gnd->g", occ, dpsi, dpsi))
    res = (torch.cat(out["rho"]),)
    if kind in ("gga", "mgga"):
        res = res + (torch.cat(out["grad"]),)
    if kind == "mgga":
        res = res + (torch.cat(out["tau"]),)
    return res

