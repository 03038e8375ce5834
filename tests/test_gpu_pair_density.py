"""The pair density q_ij = sum_o occ_o C_io C_jo of the screened passes (gs_dft/screening/pairs.py:
383-386, the DF-J and nuclear paths' pair weights), bit for bit.

The library forms each pair's sum in a fixed lane layout: G lanes per pair (G = 8, 16, 32 for
k <= 32, else 64), lane l adding (occ_o C_io) C_jo for o = l, l + G, ... in order (no fused
multiply-add), then a butterfly over the lanes (lane l adds lane l ^ off for off = G/2, ..., 1).
For 32 < k <= 2048 one wave walks a run of consecutive pairs and keeps occ_o C_io in registers while
i repeats; that must not change a bit. The replay below forms the same sums in numpy (IEEE double,
one rounding per operation) and the GPU must match it exactly: on a sorted list, where i repeats
for most of a run, and on the same pairs shuffled, where it changes at nearly every pair. The
replay is checked against a plain float64 sum to 1e-14 first, so a replay that summed the wrong
terms would fail there.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _replay(C, occ, pi, pj):
    M, k = C.shape
    G = 8 if k <= 8 else 16 if k <= 16 else 32 if k <= 32 else 64
    n = pi.shape[0]
    s = np.zeros((n, G))
    for t in range((k + G - 1) // G):
        o = np.arange(G) + G * t
        live = o < k
        oc = np.minimum(o, k - 1)
        prod = (occ[oc][None, :] * C[pi][:, oc]) * C[pj][:, oc]
        s = np.where(live[None, :], s + prod, s)
    off = G // 2
    while off > 0:
        s = s + s[:, np.arange(G) ^ off]
        off //= 2
    return s[:, 0]


@pytest.mark.parametrize("k", [5, 12, 20, 33, 81, 600, 1300, 2100])
def test_density_pairs_bit_exact_in_every_lane_layout(g, cuda, k):
    rng = np.random.default_rng(k)
    M = 257
    C = rng.normal(size=(M, k))
    occ = rng.uniform(0.0, 2.0, size=k)
    # a sorted list: each splat with a ragged run of partners (runs of the kernel straddle splats)
    pi, pj = [], []
    for i in range(M):
        for j in rng.choice(M, size=int(rng.integers(1, 9)), replace=False):
            pi.append(i)
            pj.append(int(j))
    pi, pj = np.array(pi, dtype=np.int32), np.array(pj, dtype=np.int32)
    ref = _replay(C, occ, pi, pj)
    plain = np.einsum("o,ao,ao->a", occ, C[pi], C[pj])
    scale = np.einsum("o,ao,ao->a", occ, np.abs(C[pi]), np.abs(C[pj]))
    assert np.max(np.abs(ref - plain) / scale) < 1e-14
    q = g.density_pairs(torch.tensor(C, device="cuda"), torch.tensor(occ, device="cuda"),
                        torch.tensor(pi, device="cuda"), torch.tensor(pj, device="cuda"))
    got = q.cpu().numpy()
    print(f"[density] k={k} n={pi.shape[0]} max |q - replay| = {np.max(np.abs(got - ref)):.1e}")
    assert np.array_equal(got, ref)
    perm = rng.permutation(pi.shape[0])
    qs = g.density_pairs(torch.tensor(C, device="cuda"), torch.tensor(occ, device="cuda"),
                         torch.tensor(pi[perm], device="cuda"),
                         torch.tensor(pj[perm], device="cuda")).cpu().numpy()
    assert np.array_equal(qs, ref[perm])
