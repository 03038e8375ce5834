import pathlib
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); parity tests of the HIP path")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def g():
    """The package under test (gs-dft_amd/ imported as gs_dft_amd)."""
    import __graft_entry__ as ge
    return ge.load_package()


@pytest.fixture(scope="session")
def wl(g):
    import importlib
    return importlib.import_module("gs_dft_amd.workloads")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def tr():
    from oracle import torch_ref
    return torch_ref


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device visible")
    torch.cuda.set_device(0)
    return torch.device("cuda", 0)


def rel_max(a, b):
    """max |a-b| / max |b| (0/0 -> 0)."""
    a, b = np.asarray(a, float), np.asarray(b, float)
    den = np.max(np.abs(b)) if b.size else 0.0
    if den == 0.0:
        return float(np.max(np.abs(a))) if a.size else 0.0
    return float(np.max(np.abs(a - b)) / den)
