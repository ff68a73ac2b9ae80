import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libds3_hip.so on cuda:0)")
    config.addinivalue_line("markers", "slow: long CPU oracle runs")


@pytest.fixture(scope="session")
def hip_ready():
    """Initialise the HIP backend once; GPU tests fail (not skip) if it cannot."""
    from qw3_amd import ds3
    ds3.init()
    info = ds3.device_info()
    print(f"\n[ds3_hip] device {info['arch']} CUs={info['n_cu']} HBM={info['hbm_bytes'] / 2**30:.0f} GiB", flush=True)
    return info


@pytest.fixture(scope="session")
def n_threads():
    return max(1, min(16, os.cpu_count() or 1))
