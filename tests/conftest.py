import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PACKAGE_ROOT = ROOT / "gdn-state-codec_amd"
for path in (ROOT, PACKAGE_ROOT, ROOT / "tests"):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: runs the HIP kernels on an MI355X (gfx950) GPU"
    )


@pytest.fixture(scope="session")
def device():
    """The GPU; GPU tests fail (not skip) when there is none."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but torch.cuda.is_available() is False")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    data = np.load(ROOT / "tests" / "golden" / "codec_heads.npz", allow_pickle=False)
    return {key: data[key] for key in data.files}
