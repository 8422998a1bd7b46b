import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "pulsar-asm_amd"), os.path.join(ROOT, "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long CPU oracle run")


@pytest.fixture(scope="session")
def orc():
    """The CPU oracle (test infrastructure); built here if the .so is missing."""
    import pyoracle
    if not os.path.exists(os.path.join(ROOT, "oracle", "_build", "liboracle.so")):
        import build as oracle_build  # oracle/build.py
        oracle_build.build_oracle()
    pyoracle.lib()
    return pyoracle


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def pq(dev):
    import pulsar_amd
    pulsar_amd.lib()
    return pulsar_amd
