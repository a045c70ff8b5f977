import json
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI library)")


@pytest.fixture(scope="session")
def na3d_golden():
    """{name: dict(q, k, v, out, kernel, dilation, shape)} from tests/golden/na3d_golden.npz."""
    z = np.load(GOLDEN / "na3d_golden.npz", allow_pickle=False)
    meta = json.loads(bytes(z["meta"]).decode())
    cases = {}
    for m in meta:
        n = m["name"]
        cases[n] = dict(m, q=z[f"{n}__q"], k=z[f"{n}__k"], v=z[f"{n}__v"], out=z[f"{n}__out"])
    return cases


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; fails (not skips) if the HIP library cannot be loaded there."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from strata_amd import _lib

    _lib.load()
    return torch.device("cuda:0")


def rel_l2(a, b) -> float:
    import torch

    a = a.double().cpu()
    b = b.double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))
