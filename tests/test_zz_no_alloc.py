"""gsdft_gamma_noalloc -- gsdft_gamma with its scratch in the library's static device array --
called through the C ABI against gsdft_gamma with a caller workspace: bit-identical gamma on two
calls in a row (the second on a smaller system, so it runs over the first call's leftover
scratch), agreement with the oracle, and a clean refusal of a size the scratch cannot hold."""
import ctypes

import numpy as np
import pytest
import torch

from conftest import rel_max

pytestmark = pytest.mark.gpu


def _inputs(wl, orc, s):
    la, ac = orc.product_aux(s.quat, s.log_scale, s.centers, s.scales)
    pi, pj, w, _ = orc.neighbor_pairs(s.quat, s.log_scale, s.centers, s.eps, None, True)
    d = lambda a, t=torch.float64: torch.tensor(np.ascontiguousarray(a), device="cuda", dtype=t)
    return dict(M=s.M, k=s.k, N=len(la), n=len(pi), quat=d(s.quat), ls=d(s.log_scale),
                cen=d(s.centers), C=d(s.C), occ=d(s.occ), la=d(la), ac=d(ac),
                pi=d(pi, torch.int32), pj=d(pj, torch.int32), w=d(w),
                host=(la, ac, pi, pj, w))


def _args(x):
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    return [x["M"], p(x["quat"]), p(x["ls"]), p(x["cen"]), x["k"], p(x["C"]), p(x["occ"]),
            x["N"], p(x["la"]), p(x["ac"]), x["n"], p(x["pi"]), p(x["pj"]), p(x["w"])]


def _gamma_with_workspace(_lib, x):
    L = _lib.lib()
    ws = _lib.workspace(_lib.size_query(L.gsdft_gamma_workspace_size, x["M"], x["k"], x["N"],
                                        x["n"]))
    out = torch.full((x["N"],), float("nan"), dtype=torch.float64, device="cuda")
    _lib.check(L.gsdft_gamma(*_args(x), ctypes.c_void_p(out.data_ptr()),
                             ctypes.c_void_p(ws.data_ptr()), ws.numel(), _lib.stream()),
               "gsdft_gamma")
    return out


def _gamma_noalloc(_lib, x):
    out = torch.full((x["N"],), float("nan"), dtype=torch.float64, device="cuda")
    rc = _lib.lib().gsdft_gamma_noalloc(*_args(x), ctypes.c_void_p(out.data_ptr()),
                                        _lib.stream())
    return rc, out


def test_gamma_noalloc_matches_gamma_twice_then_refuses_oversize(g, wl, orc, cuda):
    from gs_dft_amd import _lib
    for system in (2, 1):                       # the second call is the smaller system
        s = wl.make_system(system)
        x = _inputs(wl, orc, s)
        need = _lib.size_query(_lib.lib().gsdft_gamma_workspace_size, x["M"], x["k"], x["N"],
                               x["n"])
        print(f"[noalloc] system {system}: M={x['M']} N={x['N']} n={x['n']}, gsdft_gamma "
              f"workspace {need / 2**20:.1f} MiB", flush=True)
        ref = _gamma_with_workspace(_lib, x)
        rc, got = _gamma_noalloc(_lib, x)
        torch.cuda.synchronize()
        assert rc == _lib.GSDFT_OK, _lib.lib().gsdft_last_error()
        assert torch.equal(got, ref)
        la, ac, pi, pj, w = x["host"]
        go = orc.gamma(s.quat, s.log_scale, s.centers, s.C, s.occ, la, ac, pi, pj, w)
        err = rel_max(got.cpu().numpy(), go)
        print(f"[noalloc] system {system}: bit-identical to gsdft_gamma; rel {err:.2e} vs the "
              f"oracle", flush=True)
        assert err < 1e-12
    s = wl.make_system(3)                          # n = 590,298 pairs: beyond the 64 MiB
    x = _inputs(wl, orc, s)
    rc, got = _gamma_noalloc(_lib, x)
    torch.cuda.synchronize()
    msg = _lib.lib().gsdft_last_error().decode()
    print(f"[noalloc] system 3 (n={x['n']}): status {rc}: {msg}", flush=True)
    assert rc == _lib.GSDFT_ERR_ARG and "scratch" in msg
    assert bool(torch.isnan(got).all())          # nothing was launched
