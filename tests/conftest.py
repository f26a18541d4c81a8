import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(REPO, "light-interaction-project_amd")
for p in (PKG_DIR, REPO, os.path.dirname(os.path.abspath(__file__))):
    if p not in sys.path:
        sys.path.insert(0, p)

LIB = os.path.join(PKG_DIR, "li_sparse", "libli_sparse_attn.so")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); runs the HIP kernels")
    # Build the native library only when nothing is built yet.
    if not os.path.exists(LIB):
        import build_lib

        build_lib.build(jobs=4, verbose=False)


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
