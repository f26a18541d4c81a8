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
    # (Re)build the native library when it is missing or was built from other
    # sources (the hash of csrc/ and include/ recorded by the build differs).
    import build_lib

    if not build_lib.is_current():
        build_lib.build(jobs=4, verbose=False)


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
