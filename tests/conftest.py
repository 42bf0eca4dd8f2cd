import os
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: long CPU sweeps (deselect with -m 'not slow')")


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.build()
    return oracle


@pytest.fixture(scope="session")
def ref(orc):
    if not orc.ref_available():
        pytest.skip("reference build (oracle/_ref) not present")
    return orc.Ref()


@pytest.fixture(scope="session")
def gpu():
    """The HIP library on cuda:0; GPU tests fail loudly when it cannot be loaded."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but torch.cuda.is_available() is False")
    import p100_amd

    lib = p100_amd.load()
    print(f"[gpu] {torch.cuda.get_device_name(0)} lib={p100_amd.LIB_PATH}", flush=True)
    return lib


@pytest.fixture(params=["split", "mc"])
def fa_kernel(request, gpu):
    """Runs an attention test once with each first-pass kernel forced (the vector pass, and the matrix-core pass
    wherever it applies: fp16 K/V at d 128), then restores the automatic choice."""
    import p100_amd as P

    P.fa_select_kernel(request.param)
    yield request.param
    P.fa_select_kernel("auto")


GOLDEN = ROOT / "tests" / "golden"
os.environ.setdefault("OMP_NUM_THREADS", str(min(8, os.cpu_count() or 1)))
