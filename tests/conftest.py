import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "xgboost-metal_amd" / "python"))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); runs on the GPU box")
    config.addinivalue_line("markers", "slow: long CPU oracle run")


def gpu_available() -> bool:
    try:
        import ctypes
        lib = ctypes.CDLL(str(ROOT / "xgboost-metal_amd" / "python" / "xgboost" / "lib" / "libxgboost.so"))
        n = ctypes.c_int(0)
        return lib.mgb_device_count(ctypes.byref(n)) == 0 and n.value > 0
    except OSError:
        return False


@pytest.fixture(scope="session")
def xgb():
    import xgboost
    return xgboost
