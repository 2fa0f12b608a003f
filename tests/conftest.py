import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "micro-vllm_amd"), os.path.join(ROOT, "oracle"),
          os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); parity on the GPU")


@pytest.fixture(scope="session")
def orc():
    import oracle
    if not os.path.exists(oracle.ORACLE_SO):
        oracle.build(ref=False)
    return oracle.CpuMoe("oracle")


@pytest.fixture(scope="session")
def ref():
    import oracle
    if not oracle.have_ref():
        pytest.skip("oracle/_ref not built (reference tree absent)")
    return oracle.CpuMoe("ref")


@pytest.fixture(scope="session")
def hip():
    """The HIP product library on device 0; raises (never skips) if it cannot load."""
    import mvllm_hip
    mvllm_hip.init(0)
    return mvllm_hip
