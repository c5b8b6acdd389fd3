"""pytest configuration: the ``gpu`` marker and import paths.

``-m "not gpu"`` tests run on any host (oracle, host logic, library exports);
``-m gpu`` tests need an MI355X and the in-tree build of ``ascend-spmm_amd``
(they fail, not skip, when the extension is missing).
"""

import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("ascend-spmm_amd", "oracle", "tests"):
    path = os.path.join(REPO, sub)
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP extension")


@pytest.fixture(scope="session")
def spmm_npu():
    """The product module; importing it loads custom_ops_lib and libspmm_mi355x."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    import spmm_npu as module

    return module
