import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "ada-mla_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def golden():
    import numpy as np
    path = os.path.join(ROOT, "tests", "golden", "mla_ref_cpu.npz")
    with np.load(path, allow_pickle=False) as d:
        data = {k: d[k] for k in d.files}
    cases = sorted({k.split("/")[0] for k in data})
    return {c: {k.split("/")[1]: v for k, v in data.items() if k.startswith(c + "/")}
            for c in cases}
