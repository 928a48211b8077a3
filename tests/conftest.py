import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def kat():
    import numpy as np
    with np.load(GOLDEN / "litespark_kat.npz", allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.fixture(scope="session")
def forward_golden():
    import json
    import numpy as np
    with np.load(GOLDEN / "forward_tiny.npz", allow_pickle=False) as f:
        g = {k: f[k] for k in f.files}
    g["config"] = json.loads(bytes(g["config_json"]).decode())
    return g
