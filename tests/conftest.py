import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP path)")
    # Build only when nothing is built yet; the GPU box uses the prebuilt files.
    from inferno_amd import _build
    if not _build.LIB.exists():
        _build.build_hip()
    if not _build.ORACLE_LIB.exists():
        _build.build_oracle()


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
