"""The C ABI library loads and exports every entry point include/gsdft.h declares (CPU only: no
compute call is made here), and the host layer refuses to run without a GPU."""
import ctypes
import re

import pytest

from conftest import ROOT

HEADER = ROOT / "include" / "gsdft.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(gsdft_\w+)\(", text, re.M)))


@pytest.fixture(scope="module")
def built(g):
    from gs_dft_amd import _lib
    if not _lib.LIB_PATH.exists():
        import __graft_entry__ as ge
        ge.build()
    return _lib


def test_header_declares_the_entry_points():
    names = _declared()
    assert len(names) >= 20
    for must in ("gsdft_screen_build", "gsdft_gamma", "gsdft_gamma_vjp", "gsdft_cholesky",
                 "gsdft_cho_solve", "gsdft_aux_metric", "gsdft_product_aux"):
        assert must in names


def test_library_exports_every_declared_symbol(built):
    lib = ctypes.CDLL(str(built.LIB_PATH))
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_python_binding_covers_the_header(built):
    bound = set(built.SIGNATURES) | {"gsdft_last_error"}
    assert set(_declared()) == bound


def test_version_and_error_string_without_a_device(built):
    L = built.lib()
    assert L.gsdft_abi_version() == 1
    assert isinstance(L.gsdft_last_error(), bytes)


def test_no_cpu_fallback(g):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a device is visible")
    from gs_dft_amd import _lib
    with pytest.raises(_lib.GsdftError):
        g.Splat(quat=[[1.0, 0, 0, 0]], log_scale=[[0.0, 0, 0]], centers=[[0.0, 0, 0]])


def test_workspace_queries_accept_empty_inputs(built):
    """Size queries are host arithmetic (plus library size queries that may report an error
    without a GPU): an empty pair list or atom set must give a status, never a crash."""
    lib = built.lib()
    out = ctypes.c_size_t(0)
    for fn, args in ((lib.gsdft_gamma_workspace_size, (4, 1, 4, 0)),
                     (lib.gsdft_gamma_vjp_workspace_size, (4, 1, 4, 0)),
                     (lib.gsdft_gamma_vjp_workspace_size, (4, 1, 0, 0)),
                     (lib.gsdft_external_workspace_size, (4, 1, 0, 0)),
                     (lib.gsdft_external_workspace_size, (4, 1, 10, 0))):
        rc = fn(*args, ctypes.byref(out))
        assert rc in (built.GSDFT_OK, built.GSDFT_ERR_LIB, built.GSDFT_ERR_HIP)
    for sym in (0, 1):
        for grads in (0, 1):
            for n in (0, 100):
                rc = lib.gsdft_exchange_workspace_size(4, 2, 8, n, sym, grads, 0, 0,
                                                       ctypes.byref(out))
                assert rc in (built.GSDFT_OK, built.GSDFT_ERR_LIB, built.GSDFT_ERR_HIP)


def test_size_queries_refuse_lists_past_one_launch(built):
    """A one-dimensional grid holds at most 2^32 - 1 work-items and the launches over a pair list
    take up to 25 per pair, so every entry point that takes a list refuses more than 160 M pairs
    with an argument error (the size queries included, which need no GPU) instead of launching a
    grid whose size would wrap; 160 M itself is accepted by the queries. Dense arrays that one
    element-wise launch covers are held to the same bound."""
    lib = built.lib()
    out = ctypes.c_size_t(0)
    limit = 160_000_000
    queries = (lambda n: lib.gsdft_gamma_workspace_size(4, 1, 4, n, ctypes.byref(out)),
               lambda n: lib.gsdft_gamma_vjp_workspace_size(4, 1, 4, n, ctypes.byref(out)),
               lambda n: lib.gsdft_external_workspace_size(4, 1, n, 10, ctypes.byref(out)))
    for query in queries:
        assert query(limit + 1) == built.GSDFT_ERR_ARG
        assert b"pairs, more than the 160000000" in lib.gsdft_last_error()
        assert query(limit) in (built.GSDFT_OK, built.GSDFT_ERR_LIB, built.GSDFT_ERR_HIP)
    assert lib.gsdft_exact_coulomb_workspace_size(4, 1, limit + 1, 1,
                                                  ctypes.byref(out)) == built.GSDFT_ERR_ARG
    assert lib.gsdft_exchange_workspace_size(4, 2, 8, limit + 1, 1, 1, 0, 0,
                                             ctypes.byref(out)) == built.GSDFT_ERR_ARG
    # dense arrays covered by one element-wise launch: RI-K's packed columns (K2 x N_aux, here
    # 45150 x 100000 at k = 300) and the grid density's orbitals (M x k)
    assert lib.gsdft_exchange_workspace_size(2000, 300, 100000, 1000, 1, 1, 0, 0,
                                             ctypes.byref(out)) == built.GSDFT_ERR_ARG
    assert b"packed columns" in lib.gsdft_last_error()
    assert lib.gsdft_grid_density_workspace_size(3_000_000, 1500, 1024, 1, 1,
                                                 ctypes.byref(out)) == built.GSDFT_ERR_ARG
    assert b"orbitals" in lib.gsdft_last_error()


def test_pair_index_refuses_counts_past_int32(built):
    """The pair index sorts with 32-bit counts: a pair count past the int32 range is refused with
    an argument error before any library call, by the size query and by the builder itself."""
    lib = built.lib()
    out = ctypes.c_size_t(0)
    big = 2 ** 31
    assert lib.gsdft_pair_index_workspace_size(4, big, ctypes.byref(out)) == built.GSDFT_ERR_ARG
    assert b"int32" in lib.gsdft_last_error()
    dummy = ctypes.c_int32(0)
    p = ctypes.byref(dummy)
    rc = lib.gsdft_pair_index(4, big, p, p, p, p, p, p, None, 0, None)
    assert rc == built.GSDFT_ERR_ARG


def _header_params():
    """name -> list of parameter C types, parsed from include/gsdft.h."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"^\s*(?:int|const char\*)\s+(gsdft_\w+)\((.*?)\);", text, re.M | re.S):
        args = " ".join(m.group(2).split())
        if args in ("void", ""):
            out[m.group(1)] = []
            continue
        types = []
        for a in args.split(","):
            a = a.strip()
            name = re.findall(r"(\w+)$", a)[0]
            types.append(a[: -len(name)].replace(" ", ""))
        out[m.group(1)] = types
    return out


def test_ctypes_signatures_match_the_header(built):
    """Every argtypes entry of the Python binding has the width and kind of the header's
    parameter: a 32-bit int where the header says int64_t, or a missing argument, would pass
    garbage across the ABI."""
    kind = {"int64_t": ctypes.c_int64, "int": ctypes.c_int, "double": ctypes.c_double,
            "size_t": ctypes.c_size_t}
    params = _header_params()
    for name, argtypes in built.SIGNATURES.items():
        want = params[name]
        assert len(argtypes) == len(want), (name, len(argtypes), len(want))
        for k, (c, t) in enumerate(zip(want, argtypes)):
            if c.endswith("*"):
                assert t is ctypes.c_void_p or issubclass(t, ctypes._Pointer), (name, k, c, t)
                if c.rstrip("*").replace("const", "") in ("int64_t", "size_t", "double",
                                                          "uint64_t") and t is not ctypes.c_void_p:
                    base = {"int64_t": ctypes.c_int64, "size_t": ctypes.c_size_t,
                            "double": ctypes.c_double, "uint64_t": ctypes.c_uint64}
                    assert t._type_ is base[c.rstrip("*").replace("const", "")], (name, k, c, t)
            else:
                assert t is kind[c], (name, k, c, t)
