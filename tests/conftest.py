import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    import tests.helpers
    tests.helpers.CAPTURE = config.pluginmanager.getplugin("capturemanager")
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")
    config.addinivalue_line("markers", "slow: 40-layer CPU oracle measurements (minutes, ~15 GB); "
                                       "run only with FLINT_AMD_SLOW=1")


def pytest_collection_modifyitems(config, items):
    if os.environ.get("FLINT_AMD_SLOW") == "1":
        return
    skip = pytest.mark.skip(reason="40-layer CPU oracle measurement: set FLINT_AMD_SLOW=1 to run")
    for item in items:
        if "slow" in item.keywords:
            item.add_marker(skip)


def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda:0")
