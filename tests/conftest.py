import pathlib
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "llm-inference_amd" / "python"))
sys.path.insert(0, str(ROOT / "oracle"))
sys.path.insert(0, str(ROOT / "tests"))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def golden():
    def load(name):
        return np.load(GOLDEN / name, allow_pickle=False)
    return load


@pytest.fixture(scope="session")
def attn():
    import attn_mi355x
    attn_mi355x.lib()
    return attn_mi355x


@pytest.fixture(scope="session")
def gpu(attn):
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a GPU")
    name = torch.cuda.get_device_properties(0).gcnArchName
    print(f"[gpu] device 0: {name}", flush=True)
    return torch.device("cuda:0")
