import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "dgen-audio_amd"), os.path.join(ROOT, "oracle"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libdgen_hip.so on device 0)")


def _gpu_available() -> bool:
    try:
        import dgen_hip
        return dgen_hip.device_count() > 0
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """Fail loudly (not skip) when a gpu-marked test runs without a device or
    without the built library: a GPU run must exercise the HIP path."""
    import dgen_hip
    dgen_hip.load_library()
    n = dgen_hip.device_count()
    if n < 1:
        raise RuntimeError("gpu test selected but no HIP device is visible")
    return 0
