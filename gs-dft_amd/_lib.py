"""ctypes binding of ``libgsdft.so`` (the HIP/gfx950 DF-J library) and the torch plumbing.

PyTorch supplies device memory, the current stream and autograd; every computation of the DF-J
path runs in the library. There is no CPU fallback: without the built library or a GPU, every
entry point raises.
"""
from __future__ import annotations

import ctypes
import pathlib

import torch  # imported first so the library binds to the HIP runtime torch already loaded

LIB_PATH = pathlib.Path(__file__).resolve().parent / "lib" / "libgsdft.so"

GSDFT_OK = 0
GSDFT_ERR_ARG = 1
GSDFT_ERR_OVERFLOW = 2
GSDFT_ERR_NOT_PD = 3
GSDFT_ERR_HIP = 4
GSDFT_ERR_LIB = 5
GSDFT_ERR_WORKSPACE = 6
GSDFT_ERR_FALLBACK = 7

(PROF_GAMMA_FWD, PROF_GAMMA_BWD, PROF_SCREEN, PROF_METRIC, PROF_CHOLESKY, PROF_SOLVE,
 PROF_NUC_PAIRS, PROF_NUC_ATOMS, PROF_ERI_FWD, PROF_ERI_BWD, PROF_EXCH_BLOCK, PROF_EXCH_BWD,
 PROF_EXCH_TRSM, PROF_EXCH_GEMM, PROF_EXCH_SPARSE) = range(15)

_i64, _i32, _int, _dbl, _sz = ctypes.c_int64, ctypes.c_int32, ctypes.c_int, ctypes.c_double, ctypes.c_size_t
_vp = ctypes.c_void_p
_pi64 = ctypes.POINTER(ctypes.c_int64)
_psz = ctypes.POINTER(ctypes.c_size_t)
_pd = ctypes.POINTER(ctypes.c_double)

# name -> argtypes; every function returns int status except gsdft_last_error.
SIGNATURES = {
    "gsdft_abi_version": [],
    "gsdft_splat_chart": [_i64, _vp, _vp, _vp, _vp, _vp],
    "gsdft_overlap_pairs": [_i64, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _sz, _vp],
    "gsdft_screen_workspace_size": [_i64, _int, _i64, _psz],
    "gsdft_screen_count": [_i64, _vp, _vp, _vp, _dbl, _int, _vp, _sz, _pi64, _vp],
    "gsdft_screen_build": [_i64, _vp, _vp, _vp, _dbl, _int, _i64, _vp, _vp, _vp, _vp, _sz,
                           _pi64, _vp],
    "gsdft_screen_spatial_workspace_size": [_i64, _psz],
    "gsdft_screen_spatial": [_i64, _vp, _vp, _vp, _dbl, _int, _i64, _vp, _vp, _vp, _vp, _sz,
                             _pi64, _vp],
    "gsdft_pair_index_workspace_size": [_i64, _i64, _psz],
    "gsdft_pair_index": [_i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp],
    "gsdft_product_aux": [_i64, _vp, _vp, _vp, _pd, _int, _vp, _vp, _vp, _sz, _vp],
    "gsdft_product_aux_pairs": [_i64, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _pd, _int, _vp, _vp,
                                _vp, _sz, _vp],
    "gsdft_metric_workspace_size": [_i64, _psz],
    "gsdft_aux_metric": [_i64, _vp, _vp, _dbl, _dbl, _vp, _vp, _sz, _vp],
    "gsdft_cholesky": [_i64, _vp, _vp, _sz, _vp],
    "gsdft_aux_cholesky": [_i64, _vp, _vp, _dbl, _dbl, _vp, _vp, _sz, _vp],
    "gsdft_cho_solve": [_i64, _vp, _vp, _vp, _vp, _vp],
    "gsdft_gamma_workspace_size": [_i64, _i64, _i64, _i64, _psz],
    "gsdft_gamma": [_i64, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _vp, _vp,
                    _vp, _vp, _sz, _vp],
    "gsdft_gamma_noalloc": [_i64, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _vp, _i64, _vp,
                            _vp, _vp, _vp, _vp],
    "gsdft_gamma_vjp_workspace_size": [_i64, _i64, _i64, _i64, _psz],
    "gsdft_gamma_vjp": [_i64, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _vp,
                        _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz,
                        _vp],
    "gsdft_density_pairs": [_i64, _vp, _vp, _i64, _vp, _vp, _vp, _vp],
    "gsdft_external_workspace_size": [_i64, _i64, _i64, _i64, _psz],
    "gsdft_nuclear_pairs": [_i64, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _sz,
                            _vp],
    "gsdft_external_energy": [_i64, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _vp,
                              _vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                              _vp, _sz, _vp],
    "gsdft_exact_coulomb_workspace_size": [_i64, _i64, _i64, _int, _psz],
    "gsdft_exact_coulomb": [_i64, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _vp, _vp,
                            _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp],
    "gsdft_exact_coulomb_density": [_i64, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _int, _vp,
                                    _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp],
    "gsdft_dgemm": [_int, _int, _i64, _i64, _i64, _dbl, _vp, _i64, _vp, _i64, _dbl, _vp, _i64,
                    _vp],
    "gsdft_exchange_workspace_size": [_i64, _i64, _i64, _i64, _int, _int, _i64, _int, _psz],
    "gsdft_exchange": [_i64, _vp, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _vp,
                       _vp, _vp, _vp, _vp, _int, _i64, _int, _dbl, _vp, _vp, _vp, _vp, _vp, _vp,
                       _sz, _vp],
    "gsdft_grid_density_workspace_size": [_i64, _i64, _i64, _int, _int, _psz],
    "gsdft_grid_density": [_i64, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _i64, _int, _vp, _vp,
                           _vp, _vp, _sz, _vp],
    "gsdft_grid_density_vjp": [_i64, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _i64, _int, _vp,
                               _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp],
    "gsdft_profile_enable": [_int],
    "gsdft_profile_read": [_int, _pd, _pi64, _int],
    "gsdft_profile_read_work": [_int, ctypes.POINTER(ctypes.c_uint64), _int],
}

_lib = None


class GsdftError(RuntimeError):
    """A failure reported by the DF-J library."""


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise GsdftError(f"{LIB_PATH} is not built: run __graft_entry__.build() "
                             f"(hipcc --offload-arch=gfx950)")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        L.gsdft_last_error.argtypes = []
        L.gsdft_last_error.restype = ctypes.c_char_p
        _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc == GSDFT_OK:
        return
    msg = lib().gsdft_last_error().decode(errors="replace")
    if rc in (GSDFT_ERR_OVERFLOW, GSDFT_ERR_ARG):
        raise ValueError(f"{what}: {msg}")
    if rc == GSDFT_ERR_NOT_PD:
        raise torch.linalg.LinAlgError(f"{what}: {msg}")
    raise GsdftError(f"{what} failed ({rc}): {msg}")


def device() -> torch.device:
    if not torch.cuda.is_available():
        raise GsdftError("the DF-J path runs on the GPU: no HIP device is visible")
    return torch.device("cuda", torch.cuda.current_device())


def stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def f64(x, dev=None) -> torch.Tensor:
    """``x`` as a contiguous float64 tensor on the DF-J device (a copy only when needed)."""
    dev = device() if dev is None else dev
    t = x if isinstance(x, torch.Tensor) else torch.as_tensor(x)
    return t.to(device=dev, dtype=torch.float64).contiguous()


def i32(x, dev=None) -> torch.Tensor:
    dev = device() if dev is None else dev
    t = x if isinstance(x, torch.Tensor) else torch.as_tensor(x)
    return t.to(device=dev, dtype=torch.int32).contiguous()


def workspace(nbytes: int, dev=None) -> torch.Tensor:
    dev = device() if dev is None else dev
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=dev)


def size_query(fn, *args) -> int:
    out = ctypes.c_size_t(0)
    check(fn(*args, ctypes.byref(out)), fn.__name__)
    return int(out.value)


def profile_enable(on: bool = True) -> None:
    check(lib().gsdft_profile_enable(int(bool(on))), "gsdft_profile_enable")


def profile_read(kernel_id: int, reset: bool = False) -> tuple[float, int]:
    """(total milliseconds, launches) recorded for ``kernel_id`` since the last reset."""
    ms = ctypes.c_double(0.0)
    n = ctypes.c_int64(0)
    check(lib().gsdft_profile_read(int(kernel_id), ctypes.byref(ms), ctypes.byref(n),
                                   int(bool(reset))), "gsdft_profile_read")
    return float(ms.value), int(n.value)


def profile_read_work(kernel_id: int, reset: bool = False) -> int:
    """Work units executed by ``kernel_id`` while profiling was on (three-centre kernels:
    quadrature nodes evaluated over live lanes)."""
    units = ctypes.c_uint64(0)
    check(lib().gsdft_profile_read_work(int(kernel_id), ctypes.byref(units), int(bool(reset))),
          "gsdft_profile_read_work")
    return int(units.value)
