import os
import sys
from pathlib import Path

import pytest

REPO_DIR = Path(__file__).resolve().parents[1]
if str(REPO_DIR) not in sys.path:
    sys.path.insert(0, str(REPO_DIR))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: CPU test that takes more than a few seconds")


@pytest.fixture(scope="session")
def pkg():
    import __graft_entry__ as ge
    return ge.load_package()


@pytest.fixture(scope="session")
def lib(pkg):
    # FAGQ_TEST_LIBRARY: the sanitizer run (tests/test_sanitizers.py) points the
    # CPU tests at a host-sanitizer build of the same sources.
    alt = os.environ.get("FAGQ_TEST_LIBRARY")
    if alt:
        from fagq_mi355x import _lib
        _lib._lib = _lib.load(alt)
    return pkg.load_library()


@pytest.fixture(scope="session")
def gpu(pkg):
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    pkg.load_library()
    return dev


@pytest.fixture(scope="session")
def probe_lib(pkg):
    # FAGQ_TEST_PROBE_LIBRARY: the sanitizer run's build of the probe library.
    alt = os.environ.get("FAGQ_TEST_PROBE_LIBRARY")
    if alt:
        from fagq_mi355x import _lib
        _lib._probe = _lib.load_probe(alt)
    return pkg.load_probe_library()
