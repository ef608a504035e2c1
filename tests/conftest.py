import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built kernel library")


@pytest.fixture(scope="session")
def module():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from triattention_amd.kernels.extension import load_extension
    return load_extension()
