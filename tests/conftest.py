import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

# torch first: libmiq_qconv then binds to the HIP runtime torch loaded (same SONAME)
import torch  # noqa: E402,F401


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu")


@pytest.fixture(scope="session")
def device():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    lib_path = ROOT / "my_own_cnn_amd" / "libmiq_qconv.so"
    # on a GPU box the HIP library must be there: a missing build is a failure, not a skip
    assert lib_path.exists(), f"{lib_path} missing; build with python -m my_own_cnn_amd.build"
    return torch.device("cuda:0")


def pytest_report_header(config):
    return f"repo: {ROOT}  HIP_VISIBLE_DEVICES={os.environ.get('HIP_VISIBLE_DEVICES', '')}"
