import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (os.path.join(ROOT, "oracle"), os.path.join(ROOT, "edgexpu-llm_amd"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def ora():
    import oracle

    return oracle.load_oracle()


@pytest.fixture(scope="session")
def ref():
    import oracle

    r = oracle.load_reference()
    if r is None:
        pytest.skip("reference build oracle/_ref absent")
    return r


def load_golden(name: str) -> dict:
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def golden():
    return load_golden


@pytest.fixture(scope="session")
def hipdev():
    """The HIP library, initialised on cuda:0 (GPU tests only)."""
    import torch

    assert torch.cuda.is_available(), "GPU test without a GPU"
    import edgexpu_amd

    L = edgexpu_amd.hip()
    L.check(L.init(0), "init")
    return L
