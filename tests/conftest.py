"""Test configuration: the `gpu` marker and import paths.

Tests load the libraries that are already built (``python -c 'import
__graft_entry__ as g; g.build()'`` builds them); they never compile.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "npu-dialect_amd"), os.path.join(ROOT, "oracle"),
          os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu)")


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    # Load the HIP library up front so a missing build fails loudly.
    import npu_amd
    npu_amd.lib()
    return torch.device("cuda:0")
