"""Shared pytest configuration.

Marker ``gpu``: needs an MI355X (runs on the GPU box with ``-m gpu``).  Everything else
runs on the CPU here.  GPU tests call the HIP kernels through the C ABI
(``llmengine_amd.capi``) and check them against the CPU oracle (``oracle/``).
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD MI355X GPU (gfx950)")


@pytest.fixture(scope="session")
def orc():
    import oracle
    return oracle.oracle()


@pytest.fixture(scope="session")
def golden():
    import json
    with open(os.path.join(ROOT, "tests", "golden", "q8_0_golden.json")) as f:
        return json.load(f)


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected without a visible GPU")
    return torch.device("cuda:0")
