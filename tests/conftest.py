import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _ensure_oracle():
    from oracle import oracle as o
    if not os.path.exists(o.LIB_PATH):
        o.build()
    return o


@pytest.fixture(scope="session")
def orc():
    return _ensure_oracle().Oracle()


@pytest.fixture(scope="session")
def ref():
    o = _ensure_oracle()
    if not o.reference_available():
        pytest.skip("compiled reference (oracle/_ref) not available")
    r = o.Reference()
    if not r.has_avx2():
        pytest.skip("host CPU lacks AVX2/FMA for the reference build")
    return r


def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def zq():
    """The product library, initialised on the GPU; fails loudly if it cannot."""
    import zeninfer_amd.zq as z
    try:  # torch's HIP runtime first: tests mix torch tensors with the library's device calls
        import torch
        if torch.cuda.is_available():
            torch.cuda.init()
    except ImportError:
        pass
    z.lib()
    st = z.init()
    if st != 0:
        raise RuntimeError(f"zq_hip_init failed on a GPU box: {z.status_string(st)}")
    return z
