import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "strata-mlx_amd"), os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def tables():
    from strata_hip import tables as T

    t = T.synthetic(0)
    T.use(t)
    return t


HOSTRUN = os.environ.get("STRATA_HOSTRUN") == "1"


@pytest.fixture(scope="session")
def dev():
    import torch

    if HOSTRUN:
        return _host_device()
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from strata_hip import _lib

    _lib.load()  # fail loudly if the library is not built
    return torch.device("cuda:0")


def _host_device():
    """STRATA_HOSTRUN=1: the GPU tests run on the CPU against the host build of the same kernels (tests/hostrun),
    with CPU tensors standing for device memory. A check of the kernels' arithmetic and addressing where no GPU is
    at hand; the package itself only ever loads the HIP library."""
    import torch

    import hostlib
    from strata_hip import _lib

    _lib._lib = hostlib.load()

    def stream_of(t):
        if t.device.type != "cpu":
            raise ValueError(f"tensor on {t.device}: the host build takes CPU tensors")
        return None

    _lib.stream_of = stream_of
    torch.cuda.synchronize = lambda *a, **k: None
    return torch.device("cpu")


def rel_err(got, want) -> float:
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    scale = np.abs(want).max()
    return float(np.abs(got - want).max() / (scale if scale > 0 else 1.0))
