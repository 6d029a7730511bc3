import os
import sys
import tempfile
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

# Tile records written during the tests go to a throw-away store, not the
# user's; set before the package is imported (it reads the variable once).
os.environ["MM1_TUNED_STORE"] = str(Path(tempfile.mkdtemp(prefix="mm1_tiles_")) / "tiles.json")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) HIP device")


@pytest.fixture(scope="session")
def hip_device():
    import torch
    assert torch.cuda.is_available(), "GPU test run without a HIP device"
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    return torch.device("cuda:0")


@pytest.fixture(autouse=True)
def fixed_tilings(monkeypatch):
    """Kernel handles use the recorded or default tilings, never a timed
    search, so every test launches a known tiling; the tests of the search
    turn it back on themselves."""
    from mimansm1_v1_amd import attention
    monkeypatch.setattr(attention, "AUTOTUNE", False)
