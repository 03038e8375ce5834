"""The library's FP64 MFMA product (gsdft_dgemm, the dense products of the grid density and the
exchange) against numpy's on the same operands: every transpose combination, sizes that are and
are not multiples of the 128 x 128 tiles and of the 16-deep K steps, padded leading dimensions,
alpha and beta (beta = 0 must not read C, so C starts as NaN there). Bar: max |C - C_ref| within
1e-13 of max |C_ref| (round-off of K-term sums)."""
import numpy as np
import pytest
import torch

from conftest import rel_max

pytestmark = pytest.mark.gpu

CASES = [(128, 128, 128), (256, 384, 64), (1, 1, 1), (37, 300, 17), (300, 37, 129),
         (129, 257, 1000), (1300, 200, 96), (200, 1300, 48)]


def _colmajor(rng, rows, cols, ld):
    """A rows x cols column-major matrix with leading dimension ld, as a flat array."""
    buf = rng.normal(size=ld * cols)
    return buf, buf.reshape(cols, ld).T[:rows, :]


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
@pytest.mark.parametrize("m,n,k", CASES)
def test_dgemm_matches_numpy(g, cuda, ta, tb, m, n, k):
    from gs_dft_amd import _lib
    rng = np.random.default_rng(m * 7 + n * 3 + k + 11 * ta + 5 * tb)
    ar, ac = (k, m) if ta else (m, k)
    br, bc = (n, k) if tb else (k, n)
    lda, ldb, ldc = ar + 3, br + 1, m + 2
    A_buf, A = _colmajor(rng, ar, ac, lda)
    B_buf, B = _colmajor(rng, br, bc, ldb)
    opA = A.T if ta else A
    opB = B.T if tb else B
    print(f"[gemm] ta={ta} tb={tb} m={m} n={n} k={k}", flush=True)
    for alpha, beta in ((1.0, 0.0), (-2.0, 1.0), (0.5, -3.0)):
        C_buf, C = _colmajor(rng, m, n, ldc)
        ref = alpha * (opA @ opB) + (beta * C if beta != 0.0 else 0.0)
        Cd = torch.tensor(C_buf, device="cuda")
        if beta == 0.0:
            Cd.fill_(float("nan"))
        Ad, Bd = torch.tensor(A_buf, device="cuda"), torch.tensor(B_buf, device="cuda")
        _lib.check(_lib.lib().gsdft_dgemm(ta, tb, m, n, k, alpha, _lib.ptr(Ad), lda, _lib.ptr(Bd),
                                          ldb, beta, _lib.ptr(Cd), ldc, _lib.stream()), "dgemm")
        out = Cd.cpu().numpy().reshape(n, ldc).T[:m, :]
        err = rel_max(out, ref)
        assert err < 1e-13, (alpha, beta, err)
        # the padding rows of C past m are never written
        pad = Cd.cpu().numpy().reshape(n, ldc)[:, m:]
        if beta == 0.0:
            assert np.all(np.isnan(pad))
        else:
            assert np.array_equal(pad, C_buf.reshape(n, ldc)[:, m:])
